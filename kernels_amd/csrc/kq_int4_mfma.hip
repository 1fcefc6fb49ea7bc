// kq_int4_mfma.hip -- int4 group-affine GEMV / skinny GEMM on the matrix
// cores (gfx950, v_mfma_f32_16x16x32_f16).
//
// Math as in kq_int4.hip (reference int4-gemv/src/kernels.metal:17-31):
// y[b,m] = sum_g S[m,g] * (q[m,g,:] . x[b,g,:]) + B[m,g] * sum(x[b,g,:]).
//
// Why the matrix cores even at batch 1: on the vector path every 8 weights
// cost 4 AND-OR + 1 shift + 4 v_dot2 plus 64 B of LDS activation traffic;
// here the AND-OR dequant (5 VALU per 8 weights) feeds the MFMA B operand and
// the multiply-accumulate moves to the matrix pipe, whose A operand is the
// activation of at most 16 tokens (lanes of absent tokens read nothing).
//
// Operands of one MFMA (D = A.B + C, A 16x32, B 32x16):
//   A = x: lane l holds token (l%16), k-block (l/16)   -- 8 fp16 = one word
//   B = W: lane l holds row   (l%16), k-block (l/16)   -- 8 nibbles = one word
//   D[token][row]: lane l holds tokens 4*(l/16)+r, row (l%16), r < 4.
// Memory pattern: a wave instruction reads 16 rows; the run of contiguous
// bytes per row per instruction decides HBM efficiency (measured on MI355X:
// 32 B runs halve the bandwidth, 64 B runs reach ~80% of 1 KB runs). So a
// lane loads 16 B (4 words): lane group g = l/16 holds words 4g..4g+3 of a
// 128-k "span" (16 words = two 64-k quant groups A, B) -- 64 B per row per
// instruction, and the 16 waves of a workgroup take interleaved spans so the
// workgroup streams 1 KB per row. Before the MFMAs, two v_permlane32_swap
// exchange words between lanes 0-31 and 32-63 so that each lane's register t
// belongs to one group:  g0 (w0,w1,w8,w9)  g1 (w4,w5,w12,w13)
//                        g2 (w2,w3,w10,w11) g3 (w6,w7,w14,w15).
// MFMAs 0,1 (registers 0,1) then cover group A and MFMAs 2,3 group B, and the
// per-group epilogue acc += s*(D - xc) + b*xs sees pure group sums. The k
// order inside a word is the dequant order (n0,n4,n1,n5,n2,n6,n3,n7); x is
// staged in the same permuted-pair order, and each lane reads the x words
// matching its swapped registers.
//
// Work split: a persistent 1024-thread workgroup per CU walks 16-row tiles;
// wave w takes spans w, w+16, ... of the tile (split-K) in rounds of at most
// STEPS spans, issues its first loads before the x staging and the next
// round's loads before computing the current one, and the workgroup reduces
// the 16 partial tiles in LDS at the end of each tile.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kWaves = 16;
constexpr int kThreads = kWaves * 64;
constexpr int kRows = 16;  // rows per tile

struct MMeta {
    const uint16_t* S;
    const uint16_t* B;
    int bf16;
    int interleaved;
};

__device__ __forceinline__ float meta_val(uint32_t v, int bf16) {
    return bf16 ? bf2f((uint16_t)v) : h2f((uint16_t)v);
}

// LDS layout (bytes):
//   xp : [ntok][nw + 1] x 16 B   permuted pairs per word (row padded 16 B)
//   xk : [ngroups][SLOTS] float2 (sum, offset const) per token and group
//   red: [kWaves][SLOTS][kRows] float
struct Lds {
    u32x4* xp;
    float2* xk;
    float* red;
};

template <int SLOTS>
__device__ __forceinline__ Lds lds_carve(unsigned char* smem, uint32_t ntok, uint32_t nw,
                                         uint32_t ngroups) {
    Lds L;
    L.xp = reinterpret_cast<u32x4*>(smem);
    size_t off = (size_t)ntok * (nw + 1) * 16;
    L.xk = reinterpret_cast<float2*>(smem + off);
    off += (size_t)ngroups * SLOTS * 8;
    L.red = reinterpret_cast<float*>(smem + off);
    return L;
}

template <int SLOTS>
size_t lds_bytes(uint32_t ntok, uint32_t K, uint32_t G) {
    return (size_t)ntok * (K / 8 + 1) * 16 + (size_t)(K / G) * SLOTS * 8 +
           (size_t)kWaves * SLOTS * kRows * 4;
}

// Loads of one wave's part of one round: per span one 16-byte weight load and
// the span's metadata (two groups for G = 64, one for G = 128).
template <int STEPS>
struct Slice {
    u32x4 w[STEPS];
    u32x2 m[STEPS];
};

__device__ __forceinline__ uint32_t meta_word(const MMeta& mt, uint32_t mi) {
    return mt.interleaved ? reinterpret_cast<const uint32_t*>(mt.S)[mi]
                          : ((uint32_t)mt.S[mi] | ((uint32_t)mt.B[mi] << 16));
}

template <int STEPS>
__device__ __forceinline__ void load_slice(const uint32_t* __restrict__ W, const MMeta& mt,
                                           uint32_t tile, uint32_t M, uint32_t nw,
                                           uint32_t ngroups, uint32_t nspan, uint32_t i0,
                                           uint32_t n, uint32_t g64, int lane, int wave,
                                           Slice<STEPS>& sl) {
    const uint32_t row = min(tile * kRows + (lane & 15), M - 1);
    const uint32_t g = lane >> 4;
    const u32x4* wrow = reinterpret_cast<const u32x4*>(W + (size_t)row * nw);
    const uint32_t mrow = row * ngroups;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        if ((uint32_t)s < n) {
            const uint32_t span = wave + kWaves * (i0 + s);
            sl.w[s] = ldg_nt(wrow + span * 4 + g);
            if (g64) {
                sl.m[s].x = meta_word(mt, mrow + 2 * span);
                sl.m[s].y = meta_word(mt, mrow + 2 * span + 1);
            } else {
                sl.m[s].x = meta_word(mt, mrow + span);
            }
        }
    }
    (void)nspan;
}

template <int SLOTS>
__device__ __forceinline__ void epilogue(f32x4 D, uint32_t mraw, uint32_t q, const Lds& L,
                                         int bf16, uint32_t g,
                                         float (&acc)[SLOTS < 4 ? SLOTS : 4]) {
    constexpr int NR = SLOTS < 4 ? SLOTS : 4;
    const float sc = meta_val(mraw & 0xFFFFu, bf16);
    const float bi = meta_val(mraw >> 16, bf16);
    // lane groups past the token slots read slot 0 (their D is unused)
    const uint32_t slot0 = 4 * g + NR <= SLOTS ? 4 * g : 0;
    const float2* kq = L.xk + (size_t)q * SLOTS + slot0;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const float2 k2 = kq[r];
        acc[r] = fmaf(sc, D[r] - k2.y, fmaf(bi, k2.x, acc[r]));
    }
}

__device__ __forceinline__ u32x4 dequant_word(uint32_t w, const DequantConsts& kc) {
    const uint32_t w8 = w >> 8;
    return u32x4{and_or(w, kc.lo, kc.e1024), and_or(w, kc.hi, kc.e64),
                 and_or(w8, kc.lo, kc.e1024), and_or(w8, kc.hi, kc.e64)};
}

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

template <int SLOTS, int STEPS>
__device__ __forceinline__ void compute_slice(const Slice<STEPS>& sl, const Lds& L, uint32_t nw,
                                              uint32_t ntok, uint32_t i0, uint32_t n,
                                              uint32_t g64, int bf16, int lane, int wave,
                                              const DequantConsts& kc,
                                              float (&acc)[SLOTS < 4 ? SLOTS : 4]) {
    const uint32_t tok = lane & 15, g = lane >> 4;
    const bool has_tok = tok < ntok;
    // x words matching the swapped registers: (a, a+1, a+8, a+9), a = {0,4,2,6}[g]
    const uint32_t xoff = (g & 1) * 4 + (g >> 1) * 2;
    const u32x4* xrow = L.xp + (size_t)tok * (nw + 1) + xoff;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
        if ((uint32_t)s < n) {
            const uint32_t span = wave + kWaves * (i0 + s);
            u32x4 x0 = {0, 0, 0, 0}, x1 = x0, x2 = x0, x3 = x0;
            if (has_tok) {
                const u32x4* xs = xrow + span * 16;
                x0 = xs[0];
                x1 = xs[1];
                x2 = xs[8];
                x3 = xs[9];
            }
            uint32_t w0 = sl.w[s].x, w1 = sl.w[s].y, w2 = sl.w[s].z, w3 = sl.w[s].w;
            // lanes 32-63's words 0,1 <-> lanes 0-31's words 2,3
            const auto p0 = __builtin_amdgcn_permlane32_swap(w0, w2, false, false);
            const auto p1 = __builtin_amdgcn_permlane32_swap(w1, w3, false, false);
            w0 = p0[0]; w2 = p0[1];
            w1 = p1[0]; w3 = p1[1];
            if (g64) {
                f32x4 DA = mfma(x0, dequant_word(w0, kc), zero);
                DA = mfma(x1, dequant_word(w1, kc), DA);
                f32x4 DB = mfma(x2, dequant_word(w2, kc), zero);
                DB = mfma(x3, dequant_word(w3, kc), DB);
                epilogue<SLOTS>(DA, sl.m[s].x, 2 * span, L, bf16, g, acc);
                epilogue<SLOTS>(DB, sl.m[s].y, 2 * span + 1, L, bf16, g, acc);
            } else {
                f32x4 D = mfma(x0, dequant_word(w0, kc), zero);
                D = mfma(x1, dequant_word(w1, kc), D);
                D = mfma(x2, dequant_word(w2, kc), D);
                D = mfma(x3, dequant_word(w3, kc), D);
                epilogue<SLOTS>(D, sl.m[s].x, span, L, bf16, g, acc);
            }
        }
    }
}

// Stage x of ntok tokens: permuted pairs + per-group (sum, offset const).
template <int SLOTS>
__device__ __forceinline__ void stage_x(uint32_t K, uint32_t G, uint32_t ntok, const Lds& L,
                                        const u32x4 (&v)[2], uint32_t w0) {
    const uint32_t nw = K >> 3, total = ntok * nw, wpg = G >> 3;  // words per group
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t w = w0 + q * kThreads + threadIdx.x;
        float s, c;
        word_consts(v[q], s, c);
        // sum over the wpg (8 or 16) consecutive lanes holding one group
        s += dpp_f<0xB1>(s); s += dpp_f<0x4E>(s);
        c += dpp_f<0xB1>(c); c += dpp_f<0x4E>(c);
        s += __shfl_xor(s, 4, 64);
        c += __shfl_xor(c, 4, 64);
        if (wpg == 16) {
            s += __shfl_xor(s, 8, 64);
            c += __shfl_xor(c, 8, 64);
        }
        if (w < total) {
            const uint32_t t = w / nw, wi = w - t * nw;
            L.xp[(size_t)t * (nw + 1) + wi] = pair_perm(v[q]);
            if ((wi & (wpg - 1)) == 0) L.xk[(size_t)(wi / wpg) * SLOTS + t] = make_float2(s, c);
        }
    }
}

__device__ __forceinline__ void stage_load(const uint16_t* __restrict__ X, uint32_t K,
                                           uint32_t ntok, uint32_t w0, u32x4 (&v)[2]) {
    const uint32_t nw = K >> 3, total = ntok * nw;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t w = w0 + q * kThreads + threadIdx.x;
        v[q] = u32x4{0, 0, 0, 0};
        if (w < total) {
            const uint32_t t = w / nw, wi = w - t * nw;
            v[q] = *reinterpret_cast<const u32x4*>(X + (size_t)t * K + (size_t)wi * 8);
        }
    }
}

template <int SLOTS, int STEPS>
__device__ __forceinline__ void finish_tile(float (&acc)[SLOTS < 4 ? SLOTS : 4], const Lds& L,
                                            uint32_t tile, uint32_t M, uint32_t ntok,
                                            void* __restrict__ Y, int y_f32) {
    constexpr int NR = SLOTS < 4 ? SLOTS : 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t g = lane >> 4, row = lane & 15;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const uint32_t tok = 4 * g + r;
        if (tok < SLOTS) L.red[((size_t)wave * SLOTS + tok) * kRows + row] = acc[r];
        acc[r] = 0.0f;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < ntok * kRows; i += kThreads) {
        const uint32_t tok = i / kRows, rr = i % kRows, m = tile * kRows + rr;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) v += L.red[((size_t)w * SLOTS + tok) * kRows + rr];
        if (m < M) {
            const size_t o = (size_t)tok * M + m;
            if (y_f32) reinterpret_cast<float*>(Y)[o] = v;
            else reinterpret_cast<uint16_t*>(Y)[o] = f2h(v);
        }
    }
    __syncthreads();
}

// SLOTS: token slots (1, 4, 8, 16; ntok <= SLOTS). STEPS: spans a wave holds
// per work item. A work item is (tile, round); round r gives wave w the spans
// w + 16*i for i in [r*STEPS, (r+1)*STEPS). Items are double-buffered.
template <int SLOTS, int STEPS>
__global__ __launch_bounds__(kThreads) void int4_gemv_mfma(
    const uint32_t* __restrict__ W, MMeta mt, const uint16_t* __restrict__ X,
    void* __restrict__ Y, int y_f32, uint32_t M, uint32_t K, uint32_t G, uint32_t ntok) {
    constexpr int NR = SLOTS < 4 ? SLOTS : 4;
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nw = K >> 3, ngroups = K / G, nspan = K >> 7, g64 = G == 64;
    const Lds L = lds_carve<SLOTS>(smem, ntok, nw, ngroups);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t tiles = (M + kRows - 1) / kRows;
    const uint32_t mine = wave < (int)nspan ? (nspan - wave + kWaves - 1) / kWaves : 0;
    const uint32_t most = (nspan + kWaves - 1) / kWaves;
    const uint32_t rounds = (most + STEPS - 1) / STEPS;
    const uint32_t items = tiles * rounds;
    const DequantConsts kc;
    auto range = [&](uint32_t item, uint32_t& i0, uint32_t& n) {
        i0 = (item % rounds) * STEPS;
        n = i0 < mine ? min((uint32_t)STEPS, mine - i0) : 0;
    };

    float acc[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) acc[r] = 0.0f;

    // x loads first (vmcnt retires in order), then this wave's part of the
    // first item, then the staging math
    uint32_t item = blockIdx.x * rounds;
    const uint32_t stride = gridDim.x * rounds;
    const uint32_t xwords = ntok * nw;
    u32x4 xv[2];
    stage_load(X, K, ntok, 0, xv);
    Slice<STEPS> sa, sb;
    uint32_t ia = 0, na = 0, ib = 0, nb = 0;
    if (item < items) {
        range(item, ia, na);
        load_slice<STEPS>(W, mt, item / rounds, M, nw, ngroups, nspan, ia, na, g64, lane, wave, sa);
    }
    stage_x<SLOTS>(K, G, ntok, L, xv, 0);
    for (uint32_t w0 = 2 * kThreads; w0 < xwords; w0 += 2 * kThreads) {
        stage_load(X, K, ntok, w0, xv);
        stage_x<SLOTS>(K, G, ntok, L, xv, w0);
    }
    __syncthreads();

    // the items of one workgroup: its tiles' rounds in order, tiles strided
    auto next_of = [&](uint32_t it) {
        return (it % rounds) + 1 < rounds ? it + 1 : it - (it % rounds) + stride;
    };
    while (item < items) {
        uint32_t nxt = next_of(item);
        if (nxt < items) {
            range(nxt, ib, nb);
            load_slice<STEPS>(W, mt, nxt / rounds, M, nw, ngroups, nspan, ib, nb, g64, lane, wave, sb);
        }
        compute_slice<SLOTS, STEPS>(sa, L, nw, ntok, ia, na, g64, mt.bf16, lane, wave, kc, acc);
        if (item % rounds == rounds - 1)
            finish_tile<SLOTS, STEPS>(acc, L, item / rounds, M, ntok, Y, y_f32);
        item = nxt;
        if (item >= items) break;
        nxt = next_of(item);
        if (nxt < items) {
            range(nxt, ia, na);
            load_slice<STEPS>(W, mt, nxt / rounds, M, nw, ngroups, nspan, ia, na, g64, lane, wave, sa);
        }
        compute_slice<SLOTS, STEPS>(sb, L, nw, ntok, ib, nb, g64, mt.bf16, lane, wave, kc, acc);
        if (item % rounds == rounds - 1)
            finish_tile<SLOTS, STEPS>(acc, L, item / rounds, M, ntok, Y, y_f32);
        item = nxt;
    }
}

int g_ncu = 0;
int ncu() {
    if (g_ncu <= 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            g_ncu = n;
        else
            g_ncu = 256;
    }
    return g_ncu;
}

constexpr size_t kLdsMax = 160 * 1024;

uint32_t slots_for(uint32_t ntok) { return ntok <= 1 ? 1 : ntok <= 4 ? 4 : ntok <= 8 ? 8 : 16; }

uint32_t steps_needed(uint32_t K) { return ((K >> 7) + kWaves - 1) / kWaves; }

uint32_t steps_bucket(uint32_t st) { return st <= 1 ? 1 : st <= 2 ? 2 : 4; }

size_t lds_for(uint32_t slots, uint32_t ntok, uint32_t K, uint32_t G) {
    switch (slots) {
        case 1: return lds_bytes<1>(ntok, K, G);
        case 4: return lds_bytes<4>(ntok, K, G);
        case 8: return lds_bytes<8>(ntok, K, G);
        default: return lds_bytes<16>(ntok, K, G);
    }
}

// Largest token count per pass whose x stage fits the LDS.
uint32_t max_tokens(uint32_t K, uint32_t G) {
    for (uint32_t t = 16; t >= 1; --t)
        if (lds_for(slots_for(t), t, K, G) <= kLdsMax) return t;
    return 0;
}

template <int SLOTS, int STEPS>
hipError_t go(const uint32_t* W, const MMeta& mt, const uint16_t* X, void* Y, bool y_f32,
              uint32_t M, uint32_t K, uint32_t G, uint32_t ntok, hipStream_t s) {
    const size_t lds = lds_bytes<SLOTS>(ntok, K, G);
    auto kern = int4_gemv_mfma<SLOTS, STEPS>;
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
    }
    const uint32_t tiles = (M + kRows - 1) / kRows;
    const uint32_t blocks = tiles < (uint32_t)ncu() ? tiles : (uint32_t)ncu();
    kern<<<blocks, kThreads, lds, s>>>(W, mt, X, Y, y_f32 ? 1 : 0, M, K, G, ntok);
    return hipGetLastError();
}

template <int SLOTS>
hipError_t go_slots(uint32_t steps, const uint32_t* W, const MMeta& mt, const uint16_t* X,
                    void* Y, bool y_f32, uint32_t M, uint32_t K, uint32_t G, uint32_t ntok,
                    hipStream_t s) {
    switch (steps) {
        case 1: return go<SLOTS, 1>(W, mt, X, Y, y_f32, M, K, G, ntok, s);
        case 2: return go<SLOTS, 2>(W, mt, X, Y, y_f32, M, K, G, ntok, s);
        case 4: return go<SLOTS, 4>(W, mt, X, Y, y_f32, M, K, G, ntok, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

Int4Cfg int4_mfma_default(uint32_t, uint32_t, uint32_t) { return Int4Cfg{1, 1}; }

bool int4_mfma_supported(uint32_t K, uint32_t G, uint32_t batch, Int4Cfg) {
    if (batch < 1 || batch > 16) return false;
    if (!(G == 64 || G == 128) || K % 128) return false;
    return max_tokens(K, G) >= 1;
}

hipError_t launch_int4_mfma(const uint32_t* W, const uint16_t* S, const uint16_t* B, int meta_kind,
                            bool interleaved, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                            uint32_t K, uint32_t G, uint32_t batch, Int4Cfg, hipStream_t s) {
    const MMeta mt{S, B, meta_kind, interleaved ? 1 : 0};
    const uint32_t steps = steps_bucket(steps_needed(K));
    const uint32_t per_pass = max_tokens(K, G);
    const size_t ysz = y_f32 ? 4 : 2;
    for (uint32_t t0 = 0; t0 < batch;) {
        const uint32_t nt = batch - t0 < per_pass ? batch - t0 : per_pass;
        const uint16_t* Xt = X + (size_t)t0 * K;
        void* Yt = reinterpret_cast<uint8_t*>(Y) + (size_t)t0 * M * ysz;
        hipError_t e;
        switch (slots_for(nt)) {
            case 1: e = go_slots<1>(steps, W, mt, Xt, Yt, y_f32, M, K, G, nt, s); break;
            case 4: e = go_slots<4>(steps, W, mt, Xt, Yt, y_f32, M, K, G, nt, s); break;
            case 8: e = go_slots<8>(steps, W, mt, Xt, Yt, y_f32, M, K, G, nt, s); break;
            default: e = go_slots<16>(steps, W, mt, Xt, Yt, y_f32, M, K, G, nt, s); break;
        }
        if (e != hipSuccess) return e;
        t0 += nt;
    }
    return hipSuccess;
}

}  // namespace kq
