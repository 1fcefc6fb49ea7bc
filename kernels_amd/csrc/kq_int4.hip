// kq_int4.hip -- int4 group-affine GEMV, vector-ALU path (gfx950), plus the
// xsum32 and streaming-read kernels.
//
// Math (reference: int4-gemv/src/kernels.metal:17-31,397-448):
//   y[b,m] = sum_g S[m,g] * (sum_{k in g} q[m,k] x[b,k]) + B[m,g] * (sum_{k in g} x[b,k])
// evaluated per 32-weight chunk so the bias term lands exactly once per chunk.
//
// Mapping on CDNA4 (a decode GEMV is one streaming read of W):
//   * a wave instruction reads 1 KiB of one row (lane l loads 16-byte chunk
//     64*step + l): whole 128-byte lines per row, the access shape that runs
//     at the streaming-read rate (shapes with 64-byte row pieces lose ~20%);
//   * nibbles become fp16 by AND-OR into fp16 exponents (kq_device.h) and meet
//     x in v_dot2_f32_f16 (fp32 accumulation): 1 shift + 4 AND-OR + 4 dot2
//     per 8 weights and token-independent dequant; the group metadata is
//     applied once per chunk: acc += s*(d - xc) + b*xs;
//   * x is staged once per workgroup in LDS as permuted fp16 pairs
//     [token][word%4][chunk] (lane-consecutive chunks: conflict-free
//     ds_read_b128) plus per-chunk (sum, offset constant), with the chunks
//     padded to a multiple of 64 by zeros: a lane past the end of a row
//     contributes exactly 0 and no lane tests bounds. Above 8 waves only the
//     first few waves stage (about 4 words a thread) and the others issue
//     their weight loads at once: a CU's load path takes every wave's first
//     loads in turn (~7 ns a 16-byte and ~4 ns a 4-byte wave load), so the
//     fewer staging loads ahead of the weight loads, the sooner every wave's
//     first weights arrive;
//   * a workgroup of P*Q waves owns a contiguous range of row groups (R rows
//     each); wave (p, q) takes K-part p (J = steps/P consecutive steps) of row
//     groups q, q+Q, ... ("rounds"). With P = 1 a wave finishes its rows alone
//     (wave64 DPP reduction, store); with P > 1 (short matrices, to fill the
//     CUs) the P partial sums of a round meet in LDS in a fixed order;
//   * each wave streams its (row group, step) items through a ring of D
//     register slots, as deep as its items when registers allow (all of a
//     wave's loads then issue before its first compute); every load is
//     unconditional (rows are clamped to valid addresses, results discarded;
//     padding slots load out of range: zeros, no traffic) and first used by
//     the compute of its own item, and the prologue's issue order is pinned,
//     so the waitcnt pass waits for exactly one slot at a time.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kMaxWaves = 16;

struct VArgs {
    const uint32_t* W;
    const uint16_t* S;  // interleaved (scale, bias) pairs, or scales
    const uint16_t* B;  // biases (separate layout only)
    const uint16_t* X;  // [ntok][K]
    void* Y;            // [ntok][M]
    uint32_t M, K, ntok, y_f32;
    uint32_t nch, nchp, gpr, cshift;  // chunks per row (padded to 64), groups per row, log2(G/32)
    uint32_t P, Q, J;                 // K parts, row-group lanes, steps per part
    uint32_t groups_wg, ngroups;      // row groups per workgroup / in total
    uint32_t rounds, nreal, nsteps;   // rounds per workgroup; items per wave, padded to D
    uint32_t xw;                      // waves that stage x (the first xw of the workgroup)
    uint32_t pinv;                    // ceil(2^16 / P): wave / P as a multiply (exact below 16 waves)
    const uint32_t* gsel;             // gathered form: W, S, B move by gsel[0] * gstride
    uint64_t gstride;                 // bytes (one matrix of a pool, picked on the device)
};

struct VPlan {
    uint32_t R, P, Q, J, rounds, groups_wg, nwg, nreal, nsteps, D, xw;
    size_t lds;
};

template <int R, bool SB>
struct VSlot;
template <int R>
struct VSlot<R, true> {
    u32x4 w[R];
    uint32_t s[R];  // (scale | bias << 16)
};
template <int R>
struct VSlot<R, false> {
    u32x4 w[R];
    uint16_t s[R], b[R];  // widened at use: a widening next to the load would wait for it
};

template <bool BF>
__device__ __forceinline__ float mval(uint32_t v) {
    if constexpr (BF) return bf2f((uint16_t)v);
    else return h2f((uint16_t)v);
}

struct Cursor {
    uint32_t j, round;
    __device__ __forceinline__ void advance(uint32_t J) {
        if (++j == J) {
            j = 0;
            ++round;
        }
    }
};

__host__ __device__ inline size_t vlds_x(uint32_t ntok, uint32_t nchp) {
    return (size_t)ntok * nchp * 72;
}

// x in LDS: per (step s, token t) one 4608-byte block -- four planes of the
// 64 lanes' permuted pairs (plane jw = word jw of each chunk, 16 B per lane)
// and the 64 lanes' (sum, offset constant) -- at (s * NB + t) * kXBlk. A
// lane's reads of an item are one base VGPR plus immediate offsets.
constexpr uint32_t kXBlk = 4608;
constexpr int kXr = 8;  // x words a thread stages per pass (one pass up to 8 x threads)

// Register budget: a ring of R * D >= 16 row-steps, or 3-4 tokens per pass,
// needs more than 128 VGPRs, so those instantiations run at most 8 waves per
// workgroup.
template <int NB, int R, int D, bool SB, bool BF, bool GA>
__global__ __launch_bounds__(R * D >= 16 || NB >= 3 ? 512 : 1024) void int4_valu(VArgs A) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr uint32_t MB = SB ? 4 : 2;  // metadata bytes per group and array
    constexpr uint32_t kOOB = 0x80000000u;  // past every descriptor's range: loads read zeros
    const uint32_t nch = A.nch, nchp = A.nchp, nw = A.K >> 3, nstep = nchp >> 6;
    float* part = reinterpret_cast<float*>(smem + vlds_x(NB, nchp));  // [rounds][waves][R*NB]

    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const uint32_t lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t q = (wave * A.pinv) >> 16, p = wave - q * A.P;
    const uint32_t g0 = blockIdx.x * A.groups_wg;

    // Descriptors based at this workgroup's first row: every offset is small,
    // and the range checks turn the lanes past a partial last step into
    // zero loads that move no bytes.
    const uint32_t row0 = g0 * R;
    const uint32_t rows_wg = min(A.groups_wg * R, A.M - row0);
    const uint32_t rowb = A.K >> 1, metab = A.gpr * MB;
    const unsigned char* bW = reinterpret_cast<const unsigned char*>(A.W);
    const unsigned char* bS = reinterpret_cast<const unsigned char*>(A.S);
    const unsigned char* bB = reinterpret_cast<const unsigned char*>(SB ? A.S : A.B);
    if constexpr (GA) {  // one matrix of a pool, its index written by an earlier launch
        const size_t go = (size_t)__builtin_amdgcn_readfirstlane(*A.gsel) * A.gstride;
        bW += go;
        bS += go;
        bB += go;
    }
    const rsrc_t rW = make_rsrc(bW + (size_t)row0 * rowb, rows_wg * rowb);
    const rsrc_t rS = make_rsrc(bS + (size_t)row0 * metab, rows_wg * metab);
    const rsrc_t rB = make_rsrc(bB + (size_t)row0 * metab, rows_wg * metab);
    const rsrc_t rX = make_rsrc(A.X, NB * A.K * 2);

    // ---- 1. x staging loads first (vmcnt retires in order), all in one pass,
    // by the first A.xw waves only: the other waves go straight to their
    // ring loads, and no wave waits for another before its first weight load
    const uint32_t xtotal = NB * nw, xthr = A.xw * 64;
    const bool stager = wave < A.xw;  // uniform
    u32x4 sv[kXr];
    auto x_load = [&](uint32_t w0) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < kXr; ++r) {
            if (w0 + r * xthr >= xtotal) break;  // uniform
            const uint32_t w = w0 + r * xthr + tid;
            sv[r] = __builtin_amdgcn_raw_buffer_load_b128(rX, w < xtotal ? w * 16 : kOOB, 0, 0);
        }
    };
    auto x_store = [&](uint32_t w0) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < kXr; ++r) {
            if (w0 + r * xthr >= xtotal) break;  // uniform
            const uint32_t w = w0 + r * xthr + tid;
            float s, c;
            word_consts(sv[r], s, c);
            s = quad_sum(s);
            c = quad_sum(c);
            if (w < xtotal) {
                const uint32_t t = w / nw, wi = w - t * nw, ch = wi >> 2, jw = wi & 3;
                unsigned char* blk = smem + ((ch >> 6) * NB + t) * kXBlk;
                *reinterpret_cast<u32x4*>(blk + jw * 1024 + (ch & 63) * 16) = pair_perm(sv[r]);
                if (jw == 0) *reinterpret_cast<float2*>(blk + 4096 + (ch & 63) * 8) = make_float2(s, c);
            }
        }
    };
    if (stager) x_load(0);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. prime the ring
    // lane offsets: full steps, and the last step (OOB past the row's end)
    const uint32_t cl = (nstep - 1) * 64 + lane;
    const uint32_t vw_full = lane * 16, vw_last = cl < nch ? lane * 16 : kOOB;
    const uint32_t vm_full = (lane >> A.cshift) * MB, vm_last = cl < nch ? vm_full : kOOB;
    VSlot<R, SB> ring[D];
    auto issue = [&](VSlot<R, SB>& e, Cursor c) __attribute__((always_inline)) {
        // padding item (the ring depth past the wave's items): every lane
        // loads out of range, which returns zeros and moves no bytes; the
        // item's compute is skipped
        const bool pad = c.round >= A.rounds;  // uniform
        if (pad) {
            c.round = A.rounds - 1;
            c.j = A.J - 1;
        }
        // row rr of the workgroup: past its last row (the last workgroup's
        // unused row groups) every load is out of range -- zeros, no bytes
        const uint32_t s = p * A.J + c.j;
        const bool last = s == nstep - 1;
        const uint32_t vw = pad ? kOOB : last ? vw_last : vw_full;
        const uint32_t vm = pad ? kOOB : last ? vm_last : vm_full;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t rr = (c.round * A.Q + q) * R + r;
            e.w[r] = __builtin_amdgcn_raw_buffer_load_b128(rW, vw, rr * rowb + s * 1024, kNT);
            const uint32_t mo = rr * metab + (s * (64u >> A.cshift)) * MB;
            if constexpr (SB) {
                e.s[r] = __builtin_amdgcn_raw_buffer_load_b32(rS, vm, mo, 0);
            } else {
                e.s[r] = __builtin_amdgcn_raw_buffer_load_b16(rS, vm, mo, 0);
                e.b[r] = __builtin_amdgcn_raw_buffer_load_b16(rB, vm, mo, 0);
            }
        }
    };
    Cursor ci{0, 0};
#pragma unroll
    for (int d = 0; d < D; ++d) {
        issue(ring[d], ci);
        ci.advance(A.J);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 3. finish the staging, zero the padding chunks
    if (stager) {
        x_store(0);
        for (uint32_t w0 = kXr * xthr; w0 < xtotal; w0 += kXr * xthr) {
            x_load(w0);
            x_store(w0);
        }
    }
    const uint32_t npad = nchp - nch;
    for (uint32_t i = tid; i < NB * 5 * npad; i += nthr) {
        const uint32_t t = i / (5 * npad), rem = i - t * 5 * npad, jw = rem / npad;
        const uint32_t ch = nch + (rem - jw * npad);
        unsigned char* blk = smem + ((ch >> 6) * NB + t) * kXBlk;
        if (jw < 4) *reinterpret_cast<u32x4*>(blk + jw * 1024 + (ch & 63) * 16) = u32x4{0, 0, 0, 0};
        else *reinterpret_cast<float2*>(blk + 4096 + (ch & 63) * 8) = make_float2(0.0f, 0.0f);
    }
    __syncthreads();

    const DequantConsts kc;
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NB; ++t) acc[r][t] = 0.0f;

    auto store = [&](uint32_t row, int t, float v) __attribute__((always_inline)) {
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
        // K parts: this wave's partial sums of the round go to LDS; all
        // rounds are summed after the stream (one barrier per launch)
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
    const uint32_t vx_lane = lane * 16, vk_lane = 4096 + lane * 8;
    auto step = [&](const VSlot<R, SB>& e, Cursor c, uint32_t n) __attribute__((always_inline)) {
        if (n >= A.nreal) return;  // padding to the ring depth (uniform)
        const uint32_t sb = (p * A.J + c.j) * (NB * kXBlk);
        const unsigned char* bx = smem + vx_lane + sb;
        const unsigned char* bk = smem + vk_lane + sb;
        u32x4 px[NB][4];
        float2 k2[NB];
#pragma unroll
        for (int t = 0; t < NB; ++t) {
#pragma unroll
            for (int jw = 0; jw < 4; ++jw)
                px[t][jw] = *reinterpret_cast<const u32x4*>(bx + t * kXBlk + jw * 1024);
            k2[t] = *reinterpret_cast<const float2*>(bk + t * kXBlk);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32x4 d0 = dq4(e.w[r].x, kc), d1 = dq4(e.w[r].y, kc);
            const u32x4 d2 = dq4(e.w[r].z, kc), d3 = dq4(e.w[r].w, kc);
            float sc, bi;
            if constexpr (SB) {
                sc = mval<BF>(e.s[r] & 0xFFFFu);
                bi = mval<BF>(e.s[r] >> 16);
            } else {
                sc = mval<BF>(e.s[r]);
                bi = mval<BF>(e.b[r]);
            }
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const float da = dot4(d2, px[t][2], dot4(d0, px[t][0], 0.0f));
                const float db = dot4(d3, px[t][3], dot4(d1, px[t][1], 0.0f));
                acc[r][t] = fmaf(sc, (da + db) - k2[t].y, fmaf(bi, k2[t].x, acc[r][t]));
            }
        }
        if (c.j == A.J - 1) finish(c.round);
    };

    // ---- 4. main loop (loads D items ahead), then the last D items
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
    // ---- 5. K parts: sum the P partials of every round in a fixed order
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


constexpr size_t kLdsMax = 160 * 1024;
constexpr uint32_t kXwWords = 4;
// Tokens per pass of the vector path: up to 4 (x of every token of the pass
// in LDS, NB accumulators per row); a batch takes passes of 4, then 3, 2 or
// 1, each reading W once. A pass whose x does not fit LDS takes 2 tokens.
constexpr uint32_t kMaxNB = 4;

uint32_t log2u(uint32_t v) {
    uint32_t r = 0;
    while ((1u << r) < v) ++r;
    return r;
}

// Launch plan: R rows per item, P K-parts, Q row-group lanes, ring depth D.
// Measured on MI355X (Llama / 70B shapes, batch 1), the plan (1) spreads the
// row groups over every CU, (2) keeps the per-CU bytes minimal (no idle
// lanes: Q is cut to the rows a CU has), (3) among (R, P) with equal per-CU
// work, one x read shared by 2 rows and a single K part win (4096 x 14336:
// P = 1 7.7 us, P = 7 9.1 us), and (4) D = 2: deeper rings, up to all of a
// wave's items in flight at once, measured slower at every shape
// (4096 x 14336: D = 2 / 4 / 8 / 16 took 7.6 / 8.1 / 9.6 / 11.2 us;
// 14336 x 4096: 7.7 / 9.5 / 9.8 / 10.4 us). Deeper rings (forced plans
// only) cap the workgroup at 8 waves when R * D >= 16.
bool make_vplan(uint32_t M, uint32_t K, uint32_t ntok, Int4Cfg cfg, VPlan& out) {
    const uint32_t nch = K >> 5, nstep = (nch + 63) / 64, nchp = nstep * 64, cu = cu_count();
    if (cfg.unroll != 0 && cfg.unroll != 2 && cfg.unroll != 4 && cfg.unroll != 8 &&
        cfg.unroll != 16)
        return false;
    bool found = false;
    double best = 0.0;
    for (uint32_t R = 2; R >= 1; --R) {
        for (uint32_t P = 1; P <= kMaxWaves; ++P) {
            if (nstep % P) continue;
            if (cfg.rows > 0 && (uint32_t)cfg.rows != P) continue;
            const uint32_t ngroups = (M + R - 1) / R, J = nstep / P;
            const uint32_t per_cu = (ngroups + cu - 1) / cu;
            // up to 16 waves with a ring of R * D < 16 row-steps, or up to 8
            // waves with a ring of up to 16 items
            for (uint32_t wcap = kMaxWaves; wcap >= 8; wcap /= 2) {
                if (P > wcap) continue;
                if (ntok >= 3 && wcap > 8) continue;  // 8 waves at 3-4 tokens (registers)
                uint32_t dmax = wcap > 8 ? 8 / R : (ntok == 2 && R == 2 ? 8 : 16);
                if (ntok >= 3) dmax = dmax < 4 ? dmax : 4;  // 3-4 tokens: rings of 2 or 4
                if (cfg.unroll > 0 && (uint32_t)cfg.unroll > dmax) continue;
                const uint32_t qmax = wcap / P;
                const uint32_t rounds = (per_cu + qmax - 1) / qmax;
                const uint32_t Q = (per_cu + rounds - 1) / rounds;
                const uint32_t waves = P * Q, groups_wg = rounds * Q;
                const uint32_t nwg = (ngroups + groups_wg - 1) / groups_wg;
                const uint32_t nreal = rounds * J;
                const uint32_t D = cfg.unroll > 0 ? (uint32_t)cfg.unroll : 2;
                if (R * D >= 16 && waves > 8) continue;
                const uint32_t nsteps = (nreal + D - 1) / D * D;
                const size_t lds =
                    vlds_x(ntok, nchp) + (P > 1 ? (size_t)rounds * waves * R * ntok * 4 : 0);
                if (lds > kLdsMax) continue;
                // per-CU KiB plus a latency term for short waves: fewer than 8
                // waves leave HBM idle while their rings refill. At 1-2 tokens
                // not when every item of a wave is in its ring from the start:
                // more waves then only add a K-part reduction (1024 x 4096:
                // 4 waves of 2 items 2.83 us, 8 waves of 1 item in 2 parts
                // 3.00), as long as 4 waves keep every SIMD busy. At 3-4
                // tokens the compute per item triples and the term stays
                // (4097 x 1024 at 3 tokens: 5.11 us with it, 5.53 without).
                double cost = (double)nreal * waves * R;
                if (waves < 8 && (ntok >= 3 || nreal > D)) cost *= 1.0 + 0.1 * (8 - waves);
                if (waves < 4 && ntok <= 2) cost *= 1.0 + 0.1 * (4 - waves);
                // up to 16 waves: one row a wave (twice the waves of two) measured 1-3%
                // faster when a CU's rows fit in one round (4096 x 14336, 4096 x 4096)
                if (waves < 16) cost *= 1.0 + 0.005 * (16 - waves);
                // K parts: a wave finishes (reduces) its rows once per item
                // instead of once per row -- measured 4-17% slower per part count
                if (P > 1) cost *= 1.0 + 0.05 * P;
                if (R == 2) cost *= 0.98;
                if (!found || cost < best) {
                    found = true;
                    best = cost;
                    // waves that stage x: every wave up to 8; beyond that
                    // about kXwWords 16-byte words per staging thread, and
                    // the other waves issue their weight loads at once
                    // (measured against every wave staging behind a barrier:
                    // 14336 x 4096 -0.17 us, 4096 x 4096 -0.14, 4096 x 14336
                    // -0.02; with fewer staging waves each stages too much,
                    // with more the barrier's wait returns)
                    const uint32_t xwords = ntok * (K >> 3);
                    uint32_t xw = (xwords + 64 * kXwWords - 1) / (64 * kXwWords);
                    xw = waves <= 8 ? waves : xw < 1 ? 1 : xw > waves ? waves : xw;
                    out = VPlan{R, P, Q, J, rounds, groups_wg, nwg, nreal, nsteps, D, xw, lds};
                }
            }
        }
    }
    return found;
}

template <int NB, int R, int D, bool SB, bool BF, bool GA>
hipError_t vgo(const VArgs& a, const VPlan& pl, hipStream_t s) {
    auto kern = int4_valu<NB, R, D, SB, BF, GA>;
    if (pl.lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)pl.lds);
        if (e != hipSuccess) return e;
    }
    kern<<<pl.nwg, pl.P * pl.Q * 64, pl.lds, s>>>(a);
    return hipGetLastError();
}

template <int NB, int R, bool SB, bool BF, bool GA>
hipError_t vgo_d(const VArgs& a, const VPlan& pl, hipStream_t s) {
    switch (pl.D) {
        case 2: return vgo<NB, R, 2, SB, BF, GA>(a, pl, s);
        case 4: return vgo<NB, R, 4, SB, BF, GA>(a, pl, s);
        case 8:
            if constexpr (NB >= 3) return hipErrorInvalidValue;  // plans give 3-4 tokens D <= 4
            else return vgo<NB, R, 8, SB, BF, GA>(a, pl, s);
        case 16:  // two tokens on two rows: a 16-deep ring would spill
            if constexpr (NB >= 2 && R == 2) return hipErrorInvalidValue;
            else if constexpr (NB >= 3) return hipErrorInvalidValue;
            else return vgo<NB, R, 16, SB, BF, GA>(a, pl, s);
        default: return hipErrorInvalidValue;
    }
}

template <int NB, bool SB, bool BF, bool GA = false>
hipError_t vgo_r(const VArgs& a, const VPlan& pl, hipStream_t s) {
    return pl.R == 2 ? vgo_d<NB, 2, SB, BF, GA>(a, pl, s) : vgo_d<NB, 1, SB, BF, GA>(a, pl, s);
}

template <int NB>
hipError_t vgo_nb(const VArgs& a, const VPlan& pl, bool sb, bool bf, hipStream_t s) {
    if (sb) return bf ? vgo_r<NB, true, true>(a, pl, s) : vgo_r<NB, true, false>(a, pl, s);
    return bf ? vgo_r<NB, false, true>(a, pl, s) : vgo_r<NB, false, false>(a, pl, s);
}

}  // namespace

Int4Cfg int4_valu_default(uint32_t, uint32_t, uint32_t) { return Int4Cfg{0, 0}; }

// Cost of `batch` tokens on the vector path in batch-1 passes: passes of 4,
// then 3, 2 or 1 tokens (fewer where x does not fit LDS), a pass of n tokens
// costing 1, 1.12, 1.37, 1.58 (x100) batch-1 passes -- measured at 28672 x
// 8192 and 8192 x 28672 (24.9, 27.9, 34.1, 39.4 us at 1-4 tokens).
uint32_t int4_valu_cost(uint32_t M, uint32_t K, uint32_t batch) {
    static constexpr uint32_t kPass[5] = {0, 100, 112, 137, 158};
    uint32_t cost = 0;
    for (uint32_t t0 = 0; t0 < batch;) {
        uint32_t nb = batch - t0 >= kMaxNB ? kMaxNB : batch - t0;
        VPlan pl;
        while (nb > 1 && !make_vplan(M, K, nb, Int4Cfg{0, 0}, pl)) nb = nb > 2 ? 2 : 1;
        cost += kPass[nb];
        t0 += nb;
    }
    return cost;
}

// A batch-1 pass streams at ~5.3 TB/s after ~3 us of launch, ramp and tail
// (fitted: 1024x4096 .. 28672x8192 measured at 2-4 tokens, within ~15%).
double int4_valu_us(uint32_t M, uint32_t K, uint32_t G, uint32_t batch) {
    const double bytes = (double)M * K / 2 + (double)M * (K / G) * 4;
    return int4_valu_cost(M, K, batch) / 100.0 * (3.0 + bytes / 5.3e6);
}

size_t int4_valu_lds_bytes(uint32_t K, uint32_t batch) {
    const uint32_t nchp = ((K >> 5) + 63) / 64 * 64;
    return vlds_x(batch < kMaxNB ? batch : kMaxNB, nchp);
}

bool int4_valu_supported(uint32_t K, uint32_t batch, Int4Cfg cfg) {
    if (batch < 1 || batch > 16) return false;
    VPlan pl;
    return make_vplan(16, K, 1, cfg, pl);
}

hipError_t launch_int4_valu(const uint32_t* W, const uint16_t* S, const uint16_t* B, int meta_kind,
                            bool interleaved, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                            uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg, hipStream_t s,
                            const uint32_t* gsel, uint64_t gstride) {
    const size_t ysz = y_f32 ? 4 : 2;
    // the gathered form is built for the MoE expert layout: one token, split bf16 S and B
    if (gsel != nullptr && (batch != 1 || interleaved || meta_kind != 1)) return hipErrorInvalidValue;
    for (uint32_t t0 = 0; t0 < batch;) {
        uint32_t nb = batch - t0 >= kMaxNB ? kMaxNB : batch - t0;
        VPlan pl;
        while (!make_vplan(M, K, nb, cfg, pl)) {  // x of nb tokens too large for LDS
            if (nb == 1) return hipErrorInvalidValue;
            nb = nb > 2 ? 2 : 1;
        }
        VArgs a;
        a.W = W;
        a.S = S;
        a.B = B;
        a.X = X + (size_t)t0 * K;
        a.Y = reinterpret_cast<uint8_t*>(Y) + (size_t)t0 * M * ysz;
        a.M = M;
        a.K = K;
        a.ntok = nb;
        a.y_f32 = y_f32 ? 1 : 0;
        a.nch = K >> 5;
        a.nchp = ((K >> 5) + 63) / 64 * 64;
        a.gpr = K / G;
        a.cshift = log2u(G) - 5;
        a.P = pl.P;
        a.Q = pl.Q;
        a.J = pl.J;
        a.groups_wg = pl.groups_wg;
        a.ngroups = (M + pl.R - 1) / pl.R;
        a.rounds = pl.rounds;
        a.nreal = pl.nreal;
        a.nsteps = pl.nsteps;
        a.xw = pl.xw;
        a.pinv = (65536u + pl.P - 1) / pl.P;
        a.gsel = gsel;
        a.gstride = gstride;
        const bool bf = meta_kind == 1;
        const hipError_t e = gsel != nullptr ? vgo_r<1, false, true, true>(a, pl, s)
                             : nb == 4       ? vgo_nb<4>(a, pl, interleaved, bf, s)
                             : nb == 3       ? vgo_nb<3>(a, pl, interleaved, bf, s)
                             : nb == 2       ? vgo_nb<2>(a, pl, interleaved, bf, s)
                                             : vgo_nb<1>(a, pl, interleaved, bf, s);
        if (e != hipSuccess) return e;
        t0 += nb;
    }
    return hipSuccess;
}

// ---------------------------------------------------------------------------
// Debug scalar path (KQ_PATH_SCALAR), after gemv_int4_scalar (v0,
// int4-gemv/src/kernels.metal:71-95): one thread per (row, token), the row
// walked one 32-weight chunk at a time with plain loads -- d = sum q_k x_k
// and xs = sum x_k of the chunk in fp32, then acc += s * d + b * xs. No
// LDS, no shared staging, no rings: the device-side reference the fast
// paths can be checked against. Slow by design (each thread streams its own
// row).
// ---------------------------------------------------------------------------
template <int MK>
__global__ __launch_bounds__(256) void int4_scalar_k(const uint32_t* __restrict__ W,
                                                     const uint16_t* __restrict__ S,
                                                     const uint16_t* __restrict__ B, int inter,
                                                     const uint16_t* __restrict__ X, void* Y,
                                                     int yf, uint32_t M, uint32_t K, uint32_t G) {
    const uint32_t m = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (m >= M) return;
    const uint32_t groups = K / G;
    const uint32_t* w = W + (size_t)m * (K / 8);
    const uint16_t* x = X + (size_t)t * K;
    float acc = 0.0f;
    for (uint32_t c = 0; c < K / 32; ++c) {
        float d = 0.0f, xs = 0.0f;
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t p = w[c * 4 + i];
            for (uint32_t n = 0; n < 8; ++n) {
                const float xv = h2f(x[c * 32 + i * 8 + n]);
                d = fmaf((float)((p >> (4 * n)) & 0xFu), xv, d);
                xs += xv;
            }
        }
        const size_t g = (size_t)m * groups + c * 32 / G;
        const float sc = meta2f<MK>(inter ? S[2 * g] : S[g]);
        const float bs = meta2f<MK>(inter ? S[2 * g + 1] : B[g]);
        acc = fmaf(sc, d, fmaf(bs, xs, acc));
    }
    if (yf) reinterpret_cast<float*>(Y)[(size_t)t * M + m] = acc;
    else reinterpret_cast<uint16_t*>(Y)[(size_t)t * M + m] = f2h(acc);
}

hipError_t launch_int4_scalar(const uint32_t* W, const uint16_t* S, const uint16_t* B,
                              int meta_kind, bool interleaved, const uint16_t* X, void* Y,
                              bool y_f32, uint32_t M, uint32_t K, uint32_t G, uint32_t batch,
                              hipStream_t s) {
    const dim3 grid((M + 255) / 256, batch);
    if (meta_kind == 1)
        int4_scalar_k<1><<<grid, 256, 0, s>>>(W, S, B, interleaved ? 1 : 0, X, Y, y_f32 ? 1 : 0, M, K, G);
    else
        int4_scalar_k<0><<<grid, 256, 0, s>>>(W, S, B, interleaved ? 1 : 0, X, Y, y_f32 ? 1 : 0, M, K, G);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// xsum32 (int4-gemv/src/kernels.metal:54-65): one thread per 32-chunk, the
// chunk summed as eight half4 groups, each group left to right.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void xsum32_k(const uint16_t* __restrict__ X,
                                                float* __restrict__ xs, uint32_t total) {
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= total) return;
    const u32x4* p = reinterpret_cast<const u32x4*>(X) + (size_t)j * 4;
    float s = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const u32x4 v = p[q];
        s += ((h2f(v.x & 0xFFFF) + h2f(v.x >> 16)) + h2f(v.y & 0xFFFF)) + h2f(v.y >> 16);
        s += ((h2f(v.z & 0xFFFF) + h2f(v.z >> 16)) + h2f(v.w & 0xFFFF)) + h2f(v.w >> 16);
    }
    xs[j] = s;
}

hipError_t launch_xsum32(const uint16_t* X, float* xs, uint32_t K, uint32_t batch, hipStream_t s) {
    const uint32_t total = (K >> 5) * batch;
    xsum32_k<<<(total + 255) / 256, 256, 0, s>>>(X, xs, total);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Streaming-read ceiling (int4-gemv/src/kernels.metal:260-283): a grid-stride
// read, U independent 16-byte non-temporal loads per thread in flight,
// XOR-folded so the loads cannot be eliminated; the sink is written only if
// the fold is all ones. The reference's harness sweeps U and the thread
// count and keeps the best (int4-gemv/src/main.mm:294-334); so does
// bench.py. Default shape: U = 1 over 2048 x 256 threads, the best of that
// sweep on MI355X (1 GiB: 7.0 TB/s against 5.9 for U = 4 over 8192 x 256).
// With OUT, lane 0 of every wave then writes the wave's fold as a 2-byte
// value to out[w], out[w + waves], ... below nout: the read with a GEMV's
// output store, spread over the grid as a GEMV's rows are. Any launch that
// stores from every XCD pays for that at its end (the write-back of each
// XCD's dirty L2 lines), which the pure read does not.
// ---------------------------------------------------------------------------
template <int U, bool OUT>
__global__ __launch_bounds__(256) void stream_read_k(const u32x4* __restrict__ src, size_t nq,
                                                     uint32_t* __restrict__ sink,
                                                     uint16_t* __restrict__ out, uint32_t nout) {
    u32x4 a[U];
#pragma unroll
    for (int u = 0; u < U; ++u) a[u] = u32x4{0, 0, 0, 0};
    const size_t gsz = (size_t)gridDim.x * 256;
    for (size_t base = (size_t)blockIdx.x * 256 + threadIdx.x; base < nq; base += gsz * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const size_t i = base + u * gsz;
            v[u] = i < nq ? ldg_nt(src + i) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) a[u] ^= v[u];
    }
    u32x4 acc = a[0];
#pragma unroll
    for (int u = 1; u < U; ++u) acc ^= a[u];
    const uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if constexpr (OUT) {
        if ((threadIdx.x & 63) == 0) {
            const uint32_t waves = gridDim.x * 4;
            for (uint32_t o = (blockIdx.x * 256 + threadIdx.x) >> 6; o < nout; o += waves)
                out[o] = (uint16_t)(r + (r >> 16));
        }
    } else {
        if (r == 0xFFFFFFFFu) sink[0] = r;
    }
}

template <bool OUT>
hipError_t stream_read_go(const u32x4* p, size_t nq, uint32_t* sink, uint16_t* out, uint32_t nout,
                          uint32_t unroll, unsigned blocks, hipStream_t s) {
    switch (unroll) {
        case 1: stream_read_k<1, OUT><<<blocks, 256, 0, s>>>(p, nq, sink, out, nout); break;
        case 2: stream_read_k<2, OUT><<<blocks, 256, 0, s>>>(p, nq, sink, out, nout); break;
        case 4: stream_read_k<4, OUT><<<blocks, 256, 0, s>>>(p, nq, sink, out, nout); break;
        case 8: stream_read_k<8, OUT><<<blocks, 256, 0, s>>>(p, nq, sink, out, nout); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, uint32_t unroll,
                              uint32_t threads, hipStream_t s, uint16_t* out, uint32_t nout) {
    const size_t nq = bytes / 16;
    if (unroll == 0) unroll = 1;
    const unsigned blocks = threads ? threads / 256 : 2048;
    const u32x4* p = reinterpret_cast<const u32x4*>(src);
    if (out) return stream_read_go<true>(p, nq, sink, out, nout, unroll, blocks, s);
    return stream_read_go<false>(p, nq, sink, nullptr, 0, unroll, blocks, s);
}

}  // namespace kq
