// kq_int4.hip -- int4 group-affine GEMV, vector-ALU path (gfx950).
//
// Math (reference: int4-gemv/src/kernels.metal:17-31,397-448):
//   y[b,m] = sum_g S[m,g] * (sum_{k in g} q[m,k] x[b,k]) + B[m,g] * (sum_{k in g} x[b,k])
// evaluated per 32-weight chunk so the bias term lands exactly once per chunk.
//
// Mapping on CDNA4:
//   * a 256-thread workgroup stages x once into LDS as permuted fp16 pairs
//     (layout [token][word%4][chunk], 16 B per word: conflict-free
//     ds_read_b128 for lane-consecutive chunks) plus per-chunk (sum, offset
//     constant) pairs -- this replaces the reference's separate xsum32 launch;
//   * each wave owns R rows; lane l reads chunk l, l+64, ... of each row with
//     one 16-byte global load (a wave instruction covers 1 KiB of a row);
//     U such 64-chunk steps are issued before any is consumed;
//   * nibbles become fp16 by AND-OR into fp16 exponents (kq_device.h) and are
//     dotted with v_dot2_f32_f16 (fp32 accumulation); the group metadata is
//     applied once per chunk: acc += s*(d - xc) + b*xs;
//   * rows reduce with a wave64 butterfly; lane 0 stores y.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

// MK: metadata kind (0 fp16, 1 bf16). SB: interleaved (scale, bias) pairs.
template <int NB, int R, int U, int MK, bool SB>
__global__ __launch_bounds__(kThreads) void int4_gemv_valu(
    const uint32_t* __restrict__ W, const uint16_t* __restrict__ S,
    const uint16_t* __restrict__ Bm, const uint16_t* __restrict__ X, void* __restrict__ Y,
    int y_f32, uint32_t M, uint32_t K, uint32_t gshift) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nch = K >> 5;  // 32-weight chunks per row
    const uint32_t nw = K >> 3;   // packed words per row
    u32x4* xp = reinterpret_cast<u32x4*>(smem);                      // [NB][4][nch]
    float2* xk = reinterpret_cast<float2*>(smem + (size_t)NB * nch * 64);  // [NB][nch]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // ---- stage activations: permuted pairs + per-chunk (sum, offset const)
    const uint32_t total = NB * nw;
    for (uint32_t base = 0; base < total; base += kThreads) {
        const uint32_t w = base + tid;
        const bool ok = w < total;
        const uint32_t t = ok ? w / nw : 0, wi = ok ? w - t * nw : 0;
        u32x4 v = ok ? *reinterpret_cast<const u32x4*>(X + (size_t)t * K + (size_t)wi * 8)
                     : u32x4{0, 0, 0, 0};
        float s, c;
        word_consts(v, s, c);
        s = group_sum<4>(s);
        c = group_sum<4>(c);
        if (ok) {
            const uint32_t ch = wi >> 2, j = wi & 3;
            xp[(t * 4 + j) * nch + ch] = pair_perm(v);
            if (j == 0) xk[t * nch + ch] = make_float2(s, c);
        }
    }
    __syncthreads();

    const uint32_t row0 = (blockIdx.x * kWaves + wave) * R;
    if (row0 >= M) return;
    const uint32_t gpr = K >> gshift;          // groups per row
    const uint32_t cshift = gshift - 5;        // chunk -> group

    const u32x4* wrow[R];
    uint32_t mbase[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t m = min(row0 + r, M - 1);
        wrow[r] = reinterpret_cast<const u32x4*>(W + (size_t)m * nw);
        mbase[r] = m * gpr;
    }
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NB; ++t) acc[r][t] = 0.0f;

    for (uint32_t it = 0; it < nch; it += 64 * U) {
        u32x4 wv[U][R];
        uint32_t mt[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (it + 64 * u < nch) {  // wave-uniform
                const uint32_t c = min(it + 64 * u + lane, nch - 1);
                const uint32_t g = c >> cshift;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    wv[u][r] = ldg_nt(wrow[r] + c);
                    const size_t mi = (size_t)mbase[r] + g;
                    if constexpr (SB)
                        mt[u][r] = *reinterpret_cast<const uint32_t*>(S + 2 * mi);
                    else
                        mt[u][r] = (uint32_t)S[mi] | ((uint32_t)Bm[mi] << 16);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t c = it + 64 * u + lane;
            if (it + 64 * u < nch && c < nch) {
#pragma unroll
                for (int t = 0; t < NB; ++t) {
                    const u32x4 p0 = xp[(t * 4 + 0) * nch + c];
                    const u32x4 p1 = xp[(t * 4 + 1) * nch + c];
                    const u32x4 p2 = xp[(t * 4 + 2) * nch + c];
                    const u32x4 p3 = xp[(t * 4 + 3) * nch + c];
                    const float2 k2 = xk[t * nch + c];
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        const u32x4 w = wv[u][r];
                        float da = qdot8(w.x, p0, 0.0f);
                        float db = qdot8(w.y, p1, 0.0f);
                        da = qdot8(w.z, p2, da);
                        db = qdot8(w.w, p3, db);
                        const float s = meta2f<MK>(mt[u][r] & 0xFFFFu);
                        const float b = meta2f<MK>(mt[u][r] >> 16);
                        acc[r][t] = fmaf(s, (da + db) - k2.y, fmaf(b, k2.x, acc[r][t]));
                    }
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const float v = wave_sum(acc[r][t]);
            if (lane == 0 && row0 + r < M) {
                const size_t o = (size_t)t * M + row0 + r;
                if (y_f32) reinterpret_cast<float*>(Y)[o] = v;
                else reinterpret_cast<uint16_t*>(Y)[o] = f2h(v);
            }
        }
}

template <int NB, int R, int U>
hipError_t launch_nb_r_u(const uint32_t* W, const uint16_t* S, const uint16_t* B, int mk, bool sb,
                         const uint16_t* X, void* Y, bool y_f32, uint32_t M, uint32_t K,
                         uint32_t gshift, hipStream_t s) {
    const uint32_t rows_per_block = kWaves * R;
    const dim3 grid((M + rows_per_block - 1) / rows_per_block);
    const size_t lds = (size_t)NB * (K >> 5) * 72;
    if (mk == 0 && sb)
        int4_gemv_valu<NB, R, U, 0, true><<<grid, kThreads, lds, s>>>(W, S, B, X, Y, y_f32, M, K, gshift);
    else if (mk == 0)
        int4_gemv_valu<NB, R, U, 0, false><<<grid, kThreads, lds, s>>>(W, S, B, X, Y, y_f32, M, K, gshift);
    else if (sb)
        int4_gemv_valu<NB, R, U, 1, true><<<grid, kThreads, lds, s>>>(W, S, B, X, Y, y_f32, M, K, gshift);
    else
        int4_gemv_valu<NB, R, U, 1, false><<<grid, kThreads, lds, s>>>(W, S, B, X, Y, y_f32, M, K, gshift);
    return hipGetLastError();
}

template <int NB, int R>
hipError_t launch_nb_r(int U, const uint32_t* W, const uint16_t* S, const uint16_t* B, int mk,
                       bool sb, const uint16_t* X, void* Y, bool y_f32, uint32_t M, uint32_t K,
                       uint32_t gshift, hipStream_t s) {
    switch (U) {
        case 1: return launch_nb_r_u<NB, R, 1>(W, S, B, mk, sb, X, Y, y_f32, M, K, gshift, s);
        case 2: return launch_nb_r_u<NB, R, 2>(W, S, B, mk, sb, X, Y, y_f32, M, K, gshift, s);
        case 4: return launch_nb_r_u<NB, R, 4>(W, S, B, mk, sb, X, Y, y_f32, M, K, gshift, s);
        case 8: return launch_nb_r_u<NB, R, 8>(W, S, B, mk, sb, X, Y, y_f32, M, K, gshift, s);
        default: return hipErrorInvalidValue;
    }
}

template <int NB>
hipError_t launch_nb(Int4Cfg cfg, const uint32_t* W, const uint16_t* S, const uint16_t* B, int mk,
                     bool sb, const uint16_t* X, void* Y, bool y_f32, uint32_t M, uint32_t K,
                     uint32_t gshift, hipStream_t s) {
    switch (cfg.rows) {
        case 1: return launch_nb_r<NB, 1>(cfg.unroll, W, S, B, mk, sb, X, Y, y_f32, M, K, gshift, s);
        case 2: return launch_nb_r<NB, 2>(cfg.unroll, W, S, B, mk, sb, X, Y, y_f32, M, K, gshift, s);
        default: return hipErrorInvalidValue;
    }
}

uint32_t log2u(uint32_t v) {
    uint32_t r = 0;
    while ((1u << r) < v) ++r;
    return r;
}

}  // namespace

size_t int4_valu_lds_bytes(uint32_t K, uint32_t batch) { return (size_t)batch * (K >> 5) * 72; }

bool int4_valu_supported(uint32_t K, uint32_t batch, Int4Cfg cfg) {
    if (batch < 1 || batch > 16) return false;
    if (!(cfg.rows == 1 || cfg.rows == 2)) return false;
    if (!(cfg.unroll == 1 || cfg.unroll == 2 || cfg.unroll == 4 || cfg.unroll == 8)) return false;
    return int4_valu_lds_bytes(K, 1) <= 65536;
}

Int4Cfg int4_valu_default(uint32_t M, uint32_t K, uint32_t batch) {
    const uint32_t steps = ((K >> 5) + 63) / 64;
    Int4Cfg c;
    c.unroll = steps <= 1 ? 1 : steps <= 2 ? 2 : steps <= 4 ? 4 : 8;
    c.rows = (M >= 8192 && batch == 1) ? 2 : 1;
    return c;
}

hipError_t launch_int4_valu(const uint32_t* W, const uint16_t* S, const uint16_t* B, int meta_kind,
                            bool interleaved, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                            uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg, hipStream_t s) {
    const uint32_t gshift = log2u(G);
    const size_t ysz = y_f32 ? 4 : 2;
    // tokens in groups of 4, 2, 1 (each group one pass over W)
    for (uint32_t t0 = 0; t0 < batch;) {
        const uint32_t left = batch - t0;
        const uint32_t nb = (left >= 4 && int4_valu_lds_bytes(K, 4) <= 65536) ? 4
                          : (left >= 2 && int4_valu_lds_bytes(K, 2) <= 65536) ? 2 : 1;
        const uint16_t* Xt = X + (size_t)t0 * K;
        void* Yt = reinterpret_cast<uint8_t*>(Y) + (size_t)t0 * M * ysz;
        hipError_t e;
        if (nb == 4) e = launch_nb<4>(cfg, W, S, B, meta_kind, interleaved, Xt, Yt, y_f32, M, K, gshift, s);
        else if (nb == 2) e = launch_nb<2>(cfg, W, S, B, meta_kind, interleaved, Xt, Yt, y_f32, M, K, gshift, s);
        else e = launch_nb<1>(cfg, W, S, B, meta_kind, interleaved, Xt, Yt, y_f32, M, K, gshift, s);
        if (e != hipSuccess) return e;
        t0 += nb;
    }
    return hipSuccess;
}

// ---------------------------------------------------------------------------
// xsum32 (int4-gemv/src/kernels.metal:54-65): one thread per 32-chunk, the
// chunk summed as eight half4 groups, each group left to right.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void xsum32_k(const uint16_t* __restrict__ X,
                                                float* __restrict__ xs, uint32_t nch,
                                                uint32_t total) {
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
    (void)nch;
}

hipError_t launch_xsum32(const uint16_t* X, float* xs, uint32_t K, uint32_t batch, hipStream_t s) {
    const uint32_t total = (K >> 5) * batch;
    xsum32_k<<<(total + 255) / 256, 256, 0, s>>>(X, xs, K >> 5, total);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Streaming-read ceiling (int4-gemv/src/kernels.metal:260-283): U independent
// 16-byte non-temporal loads per thread in flight, XOR-folded so the loads
// cannot be eliminated; the sink is written only if the fold is all ones.
// ---------------------------------------------------------------------------
template <int U>
__global__ __launch_bounds__(256) void stream_read_k(const u32x4* __restrict__ src, size_t nq,
                                                     uint32_t* __restrict__ sink) {
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
    if (r == 0xFFFFFFFFu) sink[0] = r;
}

hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t s) {
    constexpr int U = 4;
    const size_t nq = bytes / 16;
    size_t blocks = (nq + 256 * U - 1) / (256 * U);
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    stream_read_k<U><<<(unsigned)blocks, 256, 0, s>>>(reinterpret_cast<const u32x4*>(src), nq, sink);
    return hipGetLastError();
}

}  // namespace kq
