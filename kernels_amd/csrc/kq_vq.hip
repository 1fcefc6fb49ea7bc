// kq_vq.hip -- codebook (VQ d=2, 256 entries) dequant-GEMV (gfx950).
//
// Format (reference vq-gemv/src/kernels.metal:15-27, generalised):
//   w[m, 2i+t] = S[m, 2i/scale_group] * C[m/rows_per_cb][IDX[m,i]][t]
// No bias and so no sum-of-x term (the codebook absorbs the group mean).
//
// Mapping on CDNA4 (the same skeleton as the int4 vector path, kq_int4.hip):
//   * a wave instruction reads 1 KiB of indices of one row (lane l: the
//     16-byte chunk 64*step + l = 16 indices = 32 weights);
//   * the workgroup stages x once in LDS as its natural fp16 pairs (index i
//     meets dword i of x), one 4 KiB block per (1 KiB step, token) with the
//     64 lanes' 16-byte pieces of word jw in plane jw (conflict-free
//     ds_read_b128 at immediate offsets; chunks past K zero-filled), and the
//     codebook blocks of its rows (256 x half2 = 1 KiB each);
//   * each index byte addresses one half2 codeword in LDS (ds_read_b32; one
//     of 64 interleaved copies per lane, the address one v_perm_b32),
//     dotted with its x pair by v_dot2_f32_f16 (fp32 accumulation); the
//     lookups are shared by every token of the pass; the scale applies once
//     per 32-weight chunk (scale_group % 32 == 0) or once per row;
//   * a workgroup of P*Q waves owns contiguous row groups (R rows); wave (p, q)
//     takes K-part p of row groups q, q+Q, ...; items stream through a 2-deep
//     ring of register slots with unconditional loads, the scale kept as
//     loaded until its use (so a wave waits for one slot at a time);
//   * indices and scales come with buffer loads on descriptors based at the
//     workgroup's first row (row and step offsets scalar; lanes past a
//     partial last step load out of range: zeros, no traffic); K parts meet
//     in LDS once per launch.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kMaxWaves = 16;
constexpr size_t kLdsMax = 160 * 1024;

struct QArgs {
    const uint8_t* IDX;
    const uint16_t* C;
    const uint16_t* S;
    const uint16_t* X;
    void* Y;
    uint32_t M, K, ntok, y_f32;
    uint32_t nch, nchp, rpc, spr, cshift;  // chunks, padded chunks, rows per codebook,
                                           // scales per row, chunk -> scale shift (31: per row)
    uint32_t P, Q, J, groups_wg, ngroups, rounds, nreal, nsteps;
    uint32_t cb_first_div;  // rows of a workgroup span at most this many codebooks
    uint32_t rpc_shift;     // log2(rows per codebook) if a power of 2; 31: one codebook
                            // for all rows; 32: divide
    uint32_t pinv;          // ceil(2^16 / P): wave / P as a multiply (exact below 16 waves)
};

struct QPlan {
    uint32_t R, P, Q, J, rounds, groups_wg, nwg, nreal, nsteps, D, ncb;
    size_t lds;
    uint32_t cr;  // codebook copies in LDS (kCbCopies when they fit, else 1)
};

// A lookup reads a random codebook entry per lane: with one copy, 64 random
// indices meet in the LDS banks (measured ~4 extra cycles per lookup).
// kCbCopies interleaved copies (dword e * 64 + lane) put every lane in its own
// bank, at 64 KiB per codebook block; the 256-byte entry stride makes a
// lookup's address one byte permute of the index word (vq_word_perm: 2 VALU a
// lookup instead of 3; 32 copies at a 128-byte stride took a shift and an add).
constexpr uint32_t kCbCopies = 64;
// Waves that load the codebook blocks and store their copies (16 copy groups
// of 4 copies per block, so each stores 16 / kCbStagers groups).
constexpr uint32_t kCbStagers = 4;

template <int R>
struct QSlot {
    u32x4 idx[R];
    uint16_t sc[R];  // fp16 scale bits, as loaded (widened at use)
};

struct Cursor {
    uint32_t j, round;
    __device__ __forceinline__ void advance(uint32_t J) {
        if (++j == J) {
            j = 0;
            ++round;
        }
    }
};

__host__ __device__ inline size_t qlds_x(uint32_t ntok, uint32_t nchp) {
    return (size_t)ntok * nchp * 64;
}

// One index word (4 codeword lookups) dotted with its 4 x pairs; cbr is the
// lane's copy of the codebook (CR copies interleaved by dword).
template <int CR>
__device__ __forceinline__ float vq_word(uint32_t word, u32x4 xv, const uint32_t* cbr, float acc) {
    acc = dot2(cbr[(word & 0xFF) * CR], xv.x, acc);
    acc = dot2(cbr[((word >> 8) & 0xFF) * CR], xv.y, acc);
    acc = dot2(cbr[((word >> 16) & 0xFF) * CR], xv.z, acc);
    return dot2(cbr[(word >> 24) * CR], xv.w, acc);
}
// The same with kCbCopies = 64 copies at LDS offset 0: entry e of block b,
// copy c at byte (b << 16) | (e << 8) | (c << 2), so one v_perm_b32 builds a
// lookup's address from the index byte and cbase = (b << 16) | (lane << 2)
// (byte 0 and 2 from cbase, byte 1 the index byte k of the word).
// The kernel declares no static LDS, so its dynamic area starts at LDS
// address 0 (the launcher checks that) and the address needs no base added.
__device__ __forceinline__ uint32_t lds_u32(uint32_t addr) {
    return *(const __attribute__((address_space(3))) uint32_t*)addr;
}
__device__ __forceinline__ float vq_word_perm(uint32_t word, u32x4 xv, uint32_t cbase, float acc) {
    acc = dot2(lds_u32(__builtin_amdgcn_perm(word, cbase, 0x0C020400u)), xv.x, acc);
    acc = dot2(lds_u32(__builtin_amdgcn_perm(word, cbase, 0x0C020500u)), xv.y, acc);
    acc = dot2(lds_u32(__builtin_amdgcn_perm(word, cbase, 0x0C020600u)), xv.z, acc);
    return dot2(lds_u32(__builtin_amdgcn_perm(word, cbase, 0x0C020700u)), xv.w, acc);
}

// x in LDS: per (step s, token t) one 4096-byte block of four planes (plane
// jw = word jw of each of the 64 lanes' chunks, 16 B per lane) at
// (s * NB + t) * kQBlk: a lane's reads of an item are one base VGPR plus
// immediate offsets.
constexpr uint32_t kQBlk = 4096;
constexpr int kQXr = 8;  // x words a thread stages per pass (one pass up to 8 x threads)

template <int NB, int R, int D, int CR>
__global__ __launch_bounds__(1024) void vq_valu(QArgs A) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr uint32_t kOOB = 0x80000000u;  // past every descriptor's range: loads read zeros
    const uint32_t nch = A.nch, nchp = A.nchp, nw = A.K >> 3, nstep = nchp >> 6;
    // LDS: the codebook blocks [ncb][256][CR] at offset 0, x, the K-part sums
    uint32_t* cb = reinterpret_cast<uint32_t*>(smem);
    unsigned char* xs = smem + (size_t)A.cb_first_div * 256 * CR * 4;
    float* part = reinterpret_cast<float*>(xs + qlds_x(NB, nchp));  // [rounds][waves][R*NB]

    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t q = (wave * A.pinv) >> 16, p = wave - q * A.P;
    const uint32_t g0 = blockIdx.x * A.groups_wg;
    const uint32_t last_group = A.ngroups - 1, last_row = A.M - 1;
    const uint32_t row0 = g0 * R;
    const uint32_t cb0 = row0 / A.rpc;

    // descriptors based at this workgroup's first row
    const uint32_t rows_wg = min(A.groups_wg * R, A.M - row0);
    const uint32_t rowb = A.K >> 1, srowb = A.spr * 2;
    const rsrc_t rI = make_rsrc(A.IDX + (size_t)row0 * rowb, rows_wg * rowb);
    const rsrc_t rS = make_rsrc(A.S + (size_t)row0 * A.spr, rows_wg * srowb);
    const rsrc_t rX = make_rsrc(A.X, NB * A.K * 2);

    // ---- 1. x and codebook loads first (vmcnt retires in order), then the
    // ring. Only the first waves stage: x by about ceil(words / 256) waves
    // (4 16-byte words a thread), the codebook blocks by the first
    // kCbStagers (the other waves' codebook loads fall out of range: no
    // bytes); the non-stagers issue their ring loads right after, instead of
    // behind an x load and a whole codebook block each.
    const uint32_t xtotal = NB * nw, nwv = nthr >> 6;
    const uint32_t xw = min(nwv, (xtotal + 255) / 256), xthr = xw * 64;
    const uint32_t cw = min(nwv, kCbStagers);
    const bool xst = wave < xw, cst = wave < cw;  // uniform
    u32x4 sv[kQXr];
    if (xst) {
#pragma unroll
        for (int r = 0; r < kQXr; ++r) {
            if ((uint32_t)r * xthr < xtotal) {  // uniform
                const uint32_t w = r * xthr + tid;
                sv[r] = __builtin_amdgcn_raw_buffer_load_b128(rX, w < xtotal ? w * 16 : kOOB, 0, 0);
            }
        }
    }
    // codebook blocks of this workgroup's rows (only those: the LDS area has
    // room for cb_first_div, the most any workgroup's rows can touch); with
    // CR copies, item i is entry i / (CR / 4) and stores 4 of its copies
    const uint32_t row_last = row0 + rows_wg - 1;
    const uint32_t cb_last = A.rpc_shift == 31 ? 0u
                             : A.rpc_shift < 31 ? row_last >> A.rpc_shift
                                                : row_last / A.rpc;
    const uint32_t ncb = min(A.cb_first_div, cb_last - cb0 + 1), cbn = ncb * 256;
    const uint32_t* Cw = reinterpret_cast<const uint32_t*>(A.C) + (size_t)cb0 * 256;
    // One copy: item i is entry i, a thread preloads kCbPre of them. With
    // kCbCopies (at most 2 blocks fit in LDS): every wave loads each block
    // with one 16-byte load per lane (lane l: entries 4l .. 4l + 3; the
    // second block out of range when there is one), and stores copy groups
    // of them below -- 1-2 load instructions a wave instead of the 8 that
    // 4-byte loads of (entry, copy group) items took, which delayed the
    // later waves' ring loads.
    constexpr int kCbPre = 4;
    const uint32_t cb_items = CR == 1 ? cbn : 0u;
    uint32_t cbv[kCbPre];
    u32x4 cbq[2];
    if constexpr (CR == 1) {
#pragma unroll
        for (int r = 0; r < kCbPre; ++r) {
            const uint32_t i = r * nthr + tid;
            cbv[r] = Cw[i < cb_items ? i : cbn - 1];
        }
    } else {
        // every wave issues the loads (a conditional load left the compiler
        // copying its registers, and so waiting for it, before the ring
        // loads); only the stagers' are in range
        const rsrc_t rC = make_rsrc(Cw, ncb * 1024);
#pragma unroll
        for (int b = 0; b < 2; ++b)
            cbq[b] = __builtin_amdgcn_raw_buffer_load_b128(
                rC, lane * 16 + (cst && b < (int)ncb ? b * 1024u : kOOB), 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // lane offsets: full steps, and the last step (out of range past the row)
    const uint32_t cl = (nstep - 1) * 64 + lane;
    const uint32_t vi_full = lane * 16, vi_last = cl < nch ? lane * 16 : kOOB;
    const bool per_row = A.cshift == 31;
    const uint32_t vs_full = per_row ? 0u : A.cshift <= 6 ? (lane >> A.cshift) * 2 : 0u;
    const uint32_t vs_last = cl < nch ? vs_full : kOOB;
    auto scale_step = [&](uint32_t s) __attribute__((always_inline)) {  // scale index of step s
        return per_row ? 0u : A.cshift <= 6 ? s * (64u >> A.cshift) : s >> (A.cshift - 6);
    };
    QSlot<R> ring[D];
    // padding items (the ring depth past the wave's items) and rows past the
    // workgroup's last load out of range: zeros, no bytes
    auto issue = [&](QSlot<R>& e, Cursor c) __attribute__((always_inline)) {
        const bool pad = c.round >= A.rounds;  // uniform
        if (pad) {
            c.round = A.rounds - 1;
            c.j = A.J - 1;
        }
        const uint32_t s = p * A.J + c.j;
        const bool last = s == nstep - 1;
        const uint32_t vi = pad ? kOOB : last ? vi_last : vi_full;
        const uint32_t vs = pad ? kOOB : last ? vs_last : vs_full;
        const uint32_t so = scale_step(s) * 2;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t rr = (c.round * A.Q + q) * R + r;
            e.idx[r] = __builtin_amdgcn_raw_buffer_load_b128(rI, vi, rr * rowb + s * 1024, kNT);
            e.sc[r] = __builtin_amdgcn_raw_buffer_load_b16(rS, vs, rr * srowb + so, 0);
        }
    };
    Cursor ci{0, 0};
#pragma unroll
    for (int d = 0; d < D; ++d) {
        issue(ring[d], ci);
        ci.advance(A.J);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 2. finish staging: x (as loaded: index i meets dword i), zero
    // padding, codebooks
    if (xst) {
#pragma unroll
        for (int r = 0; r < kQXr; ++r) {
            if ((uint32_t)r * xthr < xtotal) {  // uniform
                const uint32_t w = r * xthr + tid;
                if (w < xtotal) {
                    const uint32_t t = w / nw, wi = w - t * nw, ch = wi >> 2;
                    *reinterpret_cast<u32x4*>(xs + ((ch >> 6) * NB + t) * kQBlk + (wi & 3) * 1024 +
                                              (ch & 63) * 16) = sv[r];
                }
            }
        }
        for (uint32_t w0 = kQXr * xthr; w0 < xtotal; w0 += xthr) {  // past 8 words a thread
            const uint32_t w = w0 + tid;
            if (w < xtotal) {
                const uint32_t t = w / nw, wi = w - t * nw, ch = wi >> 2;
                *reinterpret_cast<u32x4*>(xs + ((ch >> 6) * NB + t) * kQBlk + (wi & 3) * 1024 +
                                          (ch & 63) * 16) = reinterpret_cast<const u32x4*>(A.X)[w];
            }
        }
    }
    const uint32_t npad = nchp - nch;
    for (uint32_t i = tid; i < NB * 4 * npad; i += nthr) {
        const uint32_t t = i / (4 * npad), rem = i - t * 4 * npad, jw = rem / npad;
        const uint32_t ch = nch + (rem - jw * npad);
        *reinterpret_cast<u32x4*>(xs + ((ch >> 6) * NB + t) * kQBlk + jw * 1024 + (ch & 63) * 16) =
            u32x4{0, 0, 0, 0};
    }
    if constexpr (CR == 1) {
#pragma unroll
        for (int r = 0; r < kCbPre; ++r) {
            const uint32_t i = r * nthr + tid;
            if (i < cb_items) cb[i] = cbv[r];
        }
        for (uint32_t i = kCbPre * nthr + tid; i < cb_items; i += nthr) cb[i] = Cw[i];
    } else {
        // copy group g = copies 4g .. 4g + 3 of an entry (16 groups). Stager
        // wave w stores groups (w' + l) % 16 of the lane's 4 entries for w' =
        // w, w + cw, ... < 16: an entry's 64 copies span the 64 banks, so the
        // 16 lanes of a quarter-wave write 16 different groups (no
        // conflicts), and over w' every (entry, group) is written once.
        static_assert(CR == 64, "copy-group stores assume 64 copies");
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (!cst || b >= (int)ncb) break;  // uniform
            const uint32_t ev[4] = {cbq[b].x, cbq[b].y, cbq[b].z, cbq[b].w};
            uint32_t* eb = cb + ((uint32_t)b * 256 + lane * 4) * CR;  // the lane's first entry
            for (uint32_t w2 = wave; w2 < 16; w2 += cw) {  // uniform
                const uint32_t g = (w2 + lane) & 15;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    *reinterpret_cast<u32x4*>(eb + k * CR + g * 4) = u32x4{ev[k], ev[k], ev[k], ev[k]};
            }
        }
    }
    __syncthreads();

    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NB; ++t) acc[r][t] = 0.0f;

    auto store = [&](uint32_t row, uint32_t t, float v) __attribute__((always_inline)) {
        const size_t o = (size_t)t * A.M + row;
        if (A.y_f32) reinterpret_cast<float*>(A.Y)[o] = v;
        else reinterpret_cast<uint16_t*>(A.Y)[o] = f2h(v);
    };
    auto finish = [&](uint32_t round) __attribute__((always_inline)) {
        const uint32_t gl = round * A.Q + q, grp = g0 + gl;
        if (A.P == 1) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    const float v = wave_sum(acc[r][t]);
                    acc[r][t] = 0.0f;
                    const uint32_t row = grp * R + r;
                    if (lane == 0 && gl < A.groups_wg && grp < A.ngroups && row < A.M)
                        store(row, t, v);
                }
            return;
        }
        // K parts: the round's partial sums wait in LDS for one reduction
        // after the stream
        float* pw = part + ((size_t)round * (A.P * A.Q) + wave) * (R * NB);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const float v = wave_sum(acc[r][t]);
                acc[r][t] = 0.0f;
                if (lane == 0) pw[r * NB + t] = v;
            }
    };
    const uint32_t rshift = A.rpc_shift;  // 31: every row uses the first block
    auto step = [&](const QSlot<R>& e, Cursor c, uint32_t n) __attribute__((always_inline)) {
        if (n >= A.nreal) return;  // padding to the ring depth (uniform)
        const unsigned char* bx = xs + lane * 16 + (p * A.J + c.j) * (NB * kQBlk);
        const uint32_t grp = min(g0 + c.round * A.Q + q, last_group);
        u32x4 xv[NB][4];
#pragma unroll
        for (int t = 0; t < NB; ++t)
#pragma unroll
            for (int w = 0; w < 4; ++w) xv[t][w] = *reinterpret_cast<const u32x4*>(bx + t * kQBlk + w * 1024);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = min(grp * R + r, last_row);
            const uint32_t blk =
                rshift == 31 ? 0u : (rshift < 31 ? row >> rshift : row / A.rpc) - cb0;  // uniform
            u32x4 iv = e.idx[r];
            uint32_t sr = e.sc[r];
            asm volatile("" : "+v"(iv), "+v"(sr));  // use the loaded values here, not earlier
            const float sc = h2f((uint16_t)sr);
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                float da, db;
                if constexpr (CR == 64) {
                    const uint32_t cbase = (blk << 16) | (lane << 2);
                    da = vq_word_perm(iv.x, xv[t][0], cbase, 0.0f);
                    db = vq_word_perm(iv.y, xv[t][1], cbase, 0.0f);
                    da = vq_word_perm(iv.z, xv[t][2], cbase, da);
                    db = vq_word_perm(iv.w, xv[t][3], cbase, db);
                } else {
                    const uint32_t* cbr = cb + blk * 256 * CR + (CR == 1 ? 0u : (lane & (CR - 1)));
                    da = vq_word<CR>(iv.x, xv[t][0], cbr, 0.0f);
                    db = vq_word<CR>(iv.y, xv[t][1], cbr, 0.0f);
                    da = vq_word<CR>(iv.z, xv[t][2], cbr, da);
                    db = vq_word<CR>(iv.w, xv[t][3], cbr, db);
                }
                acc[r][t] = fmaf(sc, da + db, acc[r][t]);
            }
        }
        if (c.j == A.J - 1) finish(c.round);
    };

    Cursor cc{0, 0};
    uint32_t n = 0;
    for (; n + D < A.nsteps; n += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            step(ring[d], cc, n + d);
            cc.advance(A.J);
            issue(ring[d], ci);
            ci.advance(A.J);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        step(ring[d], cc, n + d);
        cc.advance(A.J);
    }
    if (A.P == 1) return;
    // ---- 3. K parts: sum the P partials of every round in a fixed order
    __syncthreads();
    const uint32_t per_round = A.Q * R * NB, nout = A.rounds * per_round;
    for (uint32_t i = tid; i < nout; i += nthr) {
        const uint32_t round = i / per_round, i2 = i - round * per_round;
        const uint32_t qq = i2 / (R * NB), rt = i2 - qq * (R * NB);
        const float* pr = part + (size_t)round * (A.P * A.Q) * (R * NB);
        float v = 0.0f;
        for (uint32_t pp = 0; pp < A.P; ++pp) v += pr[(qq * A.P + pp) * (R * NB) + rt];
        const uint32_t gq = round * A.Q + qq, gg = g0 + gq, row = gg * R + rt / NB;
        if (gq < A.groups_wg && gg < A.ngroups && row < A.M) store(row, rt % NB, v);
    }
}


// Plan as for the int4 vector path (kq_int4.hip, make_vplan): spread row
// groups over every CU, no idle lanes, 2-deep ring; plus the codebook blocks a
// workgroup's rows can touch.
bool make_qplan(uint32_t M, uint32_t K, uint32_t ntok, uint32_t rpc, QPlan& out) {
    const uint32_t nch = K >> 5, nstep = (nch + 63) / 64, nchp = nstep * 64, cu = cu_count();
    bool found = false;
    double best = 0.0;
    for (uint32_t R = 2; R >= 1; --R) {
        for (uint32_t P = 1; P <= kMaxWaves; ++P) {
            if (nstep % P) continue;
            const uint32_t D = 2;
            const uint32_t ngroups = (M + R - 1) / R, J = nstep / P;
            const uint32_t per_cu = (ngroups + cu - 1) / cu;
            const uint32_t qmax = kMaxWaves / P;
            const uint32_t rounds = (per_cu + qmax - 1) / qmax;
            const uint32_t Q = (per_cu + rounds - 1) / rounds;
            const uint32_t waves = P * Q, groups_wg = rounds * Q;
            const uint32_t nwg = (ngroups + groups_wg - 1) / groups_wg;
            const uint32_t nreal = rounds * J, nsteps = (nreal + D - 1) / D * D;
            const uint32_t rows_wg = groups_wg * R;
            const uint32_t ncb = (rows_wg - 1) / rpc + 2 < (M + rpc - 1) / rpc
                                     ? (rows_wg - 1) / rpc + 2
                                     : (M + rpc - 1) / rpc;
            const size_t fixed =
                qlds_x(ntok, nchp) + (P > 1 ? (size_t)rounds * waves * R * ntok * 4 : 0);
            const size_t lds = fixed + (size_t)ncb * 1024;
            if (lds > kLdsMax) continue;
            double cost = (double)nsteps * waves * R;
            if (waves < 8) cost *= 1.0 + 0.1 * (8 - waves);
            // up to 16 waves: one row a wave (twice the waves of two) measured 1-3%
            // faster when a CU's rows fit in one round (4096 x 14336, 4096 x 4096)
            if (waves < 16) cost *= 1.0 + 0.005 * (16 - waves);
            // K parts finish (reduce) once per item instead of once per row
            if (P > 1) cost *= 1.0 + 0.05 * P;
            if (R == 2) cost *= 0.98;
            if (!found || cost < best) {
                found = true;
                best = cost;
                out = QPlan{R, P, Q, J, rounds, groups_wg, nwg, nreal, nsteps, D, ncb, lds, 1};
            }
        }
    }
    if (found) {
        const size_t rep = out.lds + (size_t)out.ncb * 1024 * (kCbCopies - 1);
        if (rep <= kLdsMax) {
            out.lds = rep;
            out.cr = kCbCopies;
        }
    }
    return found;
}

template <int NB, int R, int CR>
hipError_t qgo(const QArgs& a, const QPlan& pl, hipStream_t s) {
    auto kern = vq_valu<NB, R, 2, CR>;
    if (pl.lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)pl.lds);
        if (e != hipSuccess) return e;
    }
    kern<<<pl.nwg, pl.P * pl.Q * 64, pl.lds, s>>>(a);
    return hipGetLastError();
}

// The kCbCopies kernels address their codebooks from LDS address 0 (the
// start of the dynamic area only while the kernel has no static LDS): checked
// once per instantiation, with the one-copy kernel (same math, any LDS
// layout) in its place otherwise.
template <int NB, int R>
hipError_t qgo_copies(const QArgs& a, const QPlan& pl, hipStream_t s) {
    static const bool from_zero = [] {
        hipFuncAttributes at{};
        return hipFuncGetAttributes(&at, reinterpret_cast<const void*>(vq_valu<NB, R, 2, kCbCopies>)) ==
                   hipSuccess &&
               at.sharedSizeBytes == 0;
    }();
    return from_zero ? qgo<NB, R, kCbCopies>(a, pl, s) : qgo<NB, R, 1>(a, pl, s);
}

template <int NB>
hipError_t qgo_nb(const QArgs& a, const QPlan& pl, hipStream_t s) {
    if (pl.cr == kCbCopies) return pl.R == 2 ? qgo_copies<NB, 2>(a, pl, s) : qgo_copies<NB, 1>(a, pl, s);
    return pl.R == 2 ? qgo<NB, 2, 1>(a, pl, s) : qgo<NB, 1, 1>(a, pl, s);
}

}  // namespace

bool vq_supported(uint32_t M, uint32_t K, uint32_t rows_per_cb) {
    QPlan pl;
    return make_qplan(M, K, 1, rows_per_cb, pl);
}

hipError_t launch_vq(const uint8_t* IDX, const uint16_t* C, const uint16_t* S, const uint16_t* X,
                     void* Y, bool y_f32, uint32_t M, uint32_t K, uint32_t rows_per_cb,
                     uint32_t scale_group, uint32_t batch, hipStream_t s) {
    uint32_t sgs = 0;
    while ((1u << sgs) < scale_group) ++sgs;
    const bool per_row = scale_group == K;
    const size_t ysz = y_f32 ? 4 : 2;
    for (uint32_t t0 = 0; t0 < batch;) {
        uint32_t nb = batch - t0 >= 4 ? 4 : batch - t0 >= 2 ? 2 : 1;
        QPlan pl;
        while (!make_qplan(M, K, nb, rows_per_cb, pl)) {
            if (nb == 1) return hipErrorInvalidValue;
            nb /= 2;
        }
        QArgs a;
        a.IDX = IDX;
        a.C = C;
        a.S = S;
        a.X = X + (size_t)t0 * K;
        a.Y = reinterpret_cast<uint8_t*>(Y) + (size_t)t0 * M * ysz;
        a.M = M;
        a.K = K;
        a.ntok = nb;
        a.y_f32 = y_f32 ? 1 : 0;
        a.nch = K >> 5;
        a.nchp = ((K >> 5) + 63) / 64 * 64;
        a.rpc = rows_per_cb;
        a.spr = per_row ? 1 : K / scale_group;
        a.cshift = per_row ? 31 : sgs - 5;
        a.P = pl.P;
        a.Q = pl.Q;
        a.J = pl.J;
        a.groups_wg = pl.groups_wg;
        a.ngroups = (M + pl.R - 1) / pl.R;
        a.rounds = pl.rounds;
        a.nreal = pl.nreal;
        a.nsteps = pl.nsteps;
        a.pinv = (65536u + pl.P - 1) / pl.P;
        a.cb_first_div = pl.ncb;
        a.rpc_shift = rows_per_cb >= M ? 31u : 32u;
        if (rows_per_cb < M && (rows_per_cb & (rows_per_cb - 1)) == 0) {
            a.rpc_shift = 0;
            while ((1u << a.rpc_shift) < rows_per_cb) ++a.rpc_shift;
        }
        hipError_t e;
        if (nb == 4) e = qgo_nb<4>(a, pl, s);
        else if (nb == 2) e = qgo_nb<2>(a, pl, s);
        else e = qgo_nb<1>(a, pl, s);
        if (e != hipSuccess) return e;
        t0 += nb;
    }
    return hipSuccess;
}

}  // namespace kq
