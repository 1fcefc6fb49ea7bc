// kq_vq_quant.hip -- the VQ quantiser (gfx950): from a dense weight matrix to
// the indices, codebooks and scales kq_vq_gemv reads.
//
// Reference: quantize_matrix / _kmeans, vq-gemv/quant/pq_quantize.py:28-83
// (there an offline MLX script). Steps, each a launch (2 + 2 * iters + 1):
//
// 1. vq_scale_k: per (row, scale group) the abs-max scale (fp32), stored as
//    fp16; the pairs are normalised by the fp32 scale, 1 where it is 0
//    (pq_quantize.py:59-62).
// 2. vq_sample_k: per codebook block (rows_per_cb rows; the reference has one
//    per matrix) the k-means sample -- every pair of the block if there are
//    at most `sample`, else `sample` pairs drawn with replacement
//    (pq_quantize.py:38-39) -- and 256 initial centroids drawn from the
//    sample (pq_quantize.py:40). Draws are splitmix64 of (seed, block, draw
//    number), so a run is reproducible.
// 3. per Lloyd iteration (pq_quantize.py:41-48): vq_km_assign_k assigns each
//    sample point to argmax_c fmaf(p.x, c.x, fmaf(p.y, c.y, -|c|^2/2)) (the
//    reference's argmax of p.c - |c|^2/2; ties to the lowest c) and sums the
//    points per centroid in 2^-40 fixed point -- workgroup sums with LDS
//    atomics, then global 64-bit atomics: integer sums, so the result does
//    not depend on the order the atomics land in; vq_km_update_k moves each
//    centroid to its mean (empty clusters stay).
// 4. vq_assign_k: every pair of every row to its block's nearest fp32
//    centroid (pq_quantize.py:66-73); the codebook is stored as fp16.
//
// The assignment passes are VALU work (256 scores per pair, centroids as
// LDS broadcasts); the scale and sample passes read W once.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr uint32_t kCB = 256;   // codewords
constexpr uint32_t kQT = 256;   // threads per workgroup
constexpr uint32_t kPPT = 4;    // pairs per thread in the assignment passes
constexpr uint32_t kInitDraw = 0x80000000u;  // draw numbers of the initial centroids

struct QWs {
    size_t sc, pts, cent, acc, total;
    uint32_t ns;  // sample points per block (the stride of pts)
};

QWs qws_layout(uint32_t M, uint32_t K, uint32_t G, uint32_t R, uint32_t sample) {
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const uint32_t nblk = (M + R - 1) / R;
    const uint64_t nmax = (uint64_t)(R < M ? R : M) * (K / 2);
    QWs L;
    L.ns = (uint32_t)(nmax < sample ? nmax : sample);
    L.sc = 0;
    L.pts = al(4ull * M * (K / G));
    L.cent = L.pts + al(8ull * nblk * L.ns);
    L.acc = L.cent + al(8ull * nblk * kCB);
    L.total = L.acc + al(24ull * nblk * kCB);
    return L;
}

struct VqAcc {
    unsigned long long x, y, n;  // fixed-point sums (two's complement) and the count
};

template <int DT>
__device__ __forceinline__ float wload(const void* W, size_t i) {
    if constexpr (DT == KQ_F32) return reinterpret_cast<const float*>(W)[i];
    else if constexpr (DT == KQ_BF16) return bf2f(reinterpret_cast<const uint16_t*>(W)[i]);
    else return h2f(reinterpret_cast<const uint16_t*>(W)[i]);
}

__device__ __forceinline__ uint64_t vq_hash(uint64_t seed, uint32_t blk, uint32_t j) {
    uint64_t x = seed + 0x9E3779B97F4A7C15ull * ((((uint64_t)blk) << 32) + (uint64_t)j + 1ull);
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// uniform index in [0, n) from draw j of block blk
__device__ __forceinline__ uint32_t vq_draw(uint64_t seed, uint32_t blk, uint32_t j, uint32_t n) {
    return (uint32_t)(((vq_hash(seed, blk, j) >> 32) * (uint64_t)n) >> 32);
}

__device__ __forceinline__ float vq_hc(float cx, float cy) { return -0.5f * fmaf(cx, cx, cy * cy); }

// The normalised pair i of row m.
template <int DT>
__device__ __forceinline__ float2 vq_pair(const void* W, const float* sc, uint32_t K, uint32_t G,
                                          uint32_t m, uint32_t i) {
    const float s = sc[(size_t)m * (K / G) + (2u * i) / G];
    const size_t o = (size_t)m * K + 2u * i;
    return make_float2(wload<DT>(W, o) / s, wload<DT>(W, o + 1) / s);
}

// Sample point j of block b (every pair when the block has at most `sample`).
template <int DT>
__device__ __forceinline__ float2 vq_sample_point(const void* W, const float* sc, uint32_t K,
                                                  uint32_t G, uint32_t r0, uint32_t N,
                                                  uint32_t sample, uint64_t seed, uint32_t b,
                                                  uint32_t j) {
    const uint32_t p = N <= sample ? j : vq_draw(seed, b, j, N);
    return vq_pair<DT>(W, sc, K, G, r0 + p / (K / 2), p % (K / 2));
}

// Nearest centroid: strictly greater score wins, ascending c.
__device__ __forceinline__ uint32_t vq_nearest(float px, float py, const float4* cs) {
    uint32_t best = 0;
    float bs = -INFINITY;
    for (uint32_t c = 0; c < kCB; ++c) {
        const float4 q = cs[c];
        const float s = fmaf(px, q.x, fmaf(py, q.y, q.z));
        if (s > bs || c == 0) {
            bs = s;
            best = c;
        }
    }
    return best;
}

// Centroids of block b into LDS as (x, y, -|c|^2/2, 0).
__device__ __forceinline__ void vq_load_cent(const float2* cent, uint32_t b, float4* cs) {
    for (uint32_t c = threadIdx.x; c < kCB; c += blockDim.x) {
        const float2 v = cent[(size_t)b * kCB + c];
        cs[c] = make_float4(v.x, v.y, vq_hc(v.x, v.y), 0.0f);
    }
}

// One workgroup per row: the maxima of the row's 32-element chunks (thread
// per chunk) into LDS, then per scale group the maximum of its chunks.
template <int DT>
__global__ __launch_bounds__(kQT) void vq_scale_k(const void* __restrict__ W, uint32_t K,
                                                  uint32_t G, uint16_t* __restrict__ S,
                                                  float* __restrict__ sc) {
    extern __shared__ float cm[];  // [K / 32]
    const uint32_t m = blockIdx.x, nck = K / 32, gpr = K / G;
    const size_t row = (size_t)m * K;
    for (uint32_t c = threadIdx.x; c < nck; c += kQT) {
        float a = 0.0f;
#pragma unroll
        for (uint32_t k = 0; k < 32; ++k) a = fmaxf(a, fabsf(wload<DT>(W, row + c * 32 + k)));
        cm[c] = a;
    }
    __syncthreads();
    const uint32_t cpg = G / 32;
    for (uint32_t g = threadIdx.x; g < gpr; g += kQT) {
        float a = 0.0f;
        for (uint32_t c = 0; c < cpg; ++c) a = fmaxf(a, cm[g * cpg + c]);
        S[(size_t)m * gpr + g] = f2h(a);
        sc[(size_t)m * gpr + g] = a > 0.0f ? a : 1.0f;
    }
}

template <int DT>
__global__ __launch_bounds__(kQT) void vq_sample_k(const void* __restrict__ W, uint32_t M,
                                                   uint32_t K, uint32_t G, uint32_t R,
                                                   uint32_t sample, uint32_t ns_stride,
                                                   uint64_t seed, const float* __restrict__ sc,
                                                   float2* __restrict__ pts,
                                                   float2* __restrict__ cent,
                                                   uint16_t* __restrict__ Cb,
                                                   VqAcc* __restrict__ acc) {
    const uint32_t b = blockIdx.y, r0 = b * R, rows = min(R, M - r0);
    const uint32_t N = rows * (K / 2), ns = min(N, sample);
    const uint32_t j = blockIdx.x * kQT + threadIdx.x;
    if (j < ns)
        pts[(size_t)b * ns_stride + j] =
            vq_sample_point<DT>(W, sc, K, G, r0, N, sample, seed, b, j);
    if (blockIdx.x == 0) {
        for (uint32_t c = threadIdx.x; c < kCB; c += kQT) {
            const uint32_t jj = vq_draw(seed, b, kInitDraw + c, ns);
            const float2 v = vq_sample_point<DT>(W, sc, K, G, r0, N, sample, seed, b, jj);
            cent[(size_t)b * kCB + c] = v;
            Cb[((size_t)b * kCB + c) * 2] = f2h(v.x);
            Cb[((size_t)b * kCB + c) * 2 + 1] = f2h(v.y);
            acc[(size_t)b * kCB + c] = VqAcc{0, 0, 0};
        }
    }
}

__global__ __launch_bounds__(kQT) void vq_km_assign_k(const float2* __restrict__ pts,
                                                      uint32_t ns_stride, uint32_t M, uint32_t K,
                                                      uint32_t R, uint32_t sample,
                                                      const float2* __restrict__ cent,
                                                      VqAcc* __restrict__ acc) {
    __shared__ float4 cs[kCB];
    __shared__ unsigned long long sx[kCB], sy[kCB], sn[kCB];
    const uint32_t b = blockIdx.y, rows = min(R, M - b * R);
    const uint32_t ns = min(rows * (K / 2), sample);
    const uint32_t j0 = blockIdx.x * kQT * kPPT;
    if (j0 >= ns) return;  // uniform
    vq_load_cent(cent, b, cs);
    for (uint32_t c = threadIdx.x; c < kCB; c += kQT) sx[c] = sy[c] = sn[c] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t u = 0; u < kPPT; ++u) {
        const uint32_t j = j0 + u * kQT + threadIdx.x;
        if (j < ns) {
            const float2 p = pts[(size_t)b * ns_stride + j];
            const uint32_t a = vq_nearest(p.x, p.y, cs);
            atomicAdd(&sx[a], (unsigned long long)__float2ll_rz(p.x * 0x1p40f));
            atomicAdd(&sy[a], (unsigned long long)__float2ll_rz(p.y * 0x1p40f));
            atomicAdd(&sn[a], 1ull);
        }
    }
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < kCB; c += kQT) {
        if (sn[c] == 0) continue;
        VqAcc* q = acc + (size_t)b * kCB + c;
        atomicAdd(&q->x, sx[c]);
        atomicAdd(&q->y, sy[c]);
        atomicAdd(&q->n, sn[c]);
    }
}

__global__ __launch_bounds__(kQT) void vq_km_update_k(VqAcc* __restrict__ acc,
                                                      float2* __restrict__ cent,
                                                      uint16_t* __restrict__ Cb) {
    const size_t i = (size_t)blockIdx.x * kCB + threadIdx.x;
    const VqAcc q = acc[i];
    if (q.n != 0) {
        const float2 v = make_float2((float)((double)(long long)q.x * 0x1p-40 / (double)q.n),
                                     (float)((double)(long long)q.y * 0x1p-40 / (double)q.n));
        cent[i] = v;
        Cb[2 * i] = f2h(v.x);
        Cb[2 * i + 1] = f2h(v.y);
    }
    acc[i] = VqAcc{0, 0, 0};
}

// One workgroup per (row, kQT * kPPT pairs) (grid x = rows); thread t takes pairs 4t .. 4t+3
// of the workgroup's range and writes their 4 index bytes as one word.
template <int DT>
__global__ __launch_bounds__(kQT) void vq_assign_k(const void* __restrict__ W, uint32_t K,
                                                   uint32_t G, uint32_t R,
                                                   const float* __restrict__ sc,
                                                   const float2* __restrict__ cent,
                                                   uint8_t* __restrict__ IDX) {
    __shared__ float4 cs[kCB];
    const uint32_t m = blockIdx.x, half = K / 2;
    vq_load_cent(cent, m / R, cs);
    __syncthreads();
    const uint32_t i0 = (blockIdx.y * kQT + threadIdx.x) * kPPT;
    if (i0 >= half) return;
    uint32_t word = 0;
#pragma unroll
    for (uint32_t u = 0; u < kPPT; ++u) {
        const float2 p = vq_pair<DT>(W, sc, K, G, m, i0 + u);
        word |= vq_nearest(p.x, p.y, cs) << (8 * u);
    }
    *reinterpret_cast<uint32_t*>(IDX + (size_t)m * half + i0) = word;
}

template <int DT>
hipError_t vq_quant_go(const void* W, uint32_t M, uint32_t K, uint32_t G, uint32_t R,
                       uint32_t iters, uint32_t sample, uint64_t seed, uint8_t* IDX, uint16_t* Cb,
                       uint16_t* S, uint8_t* ws, hipStream_t s) {
    const QWs L = qws_layout(M, K, G, R, sample);
    float* sc = reinterpret_cast<float*>(ws + L.sc);
    float2* pts = reinterpret_cast<float2*>(ws + L.pts);
    float2* cent = reinterpret_cast<float2*>(ws + L.cent);
    VqAcc* acc = reinterpret_cast<VqAcc*>(ws + L.acc);
    const uint32_t nblk = (M + R - 1) / R;
    vq_scale_k<DT><<<M, kQT, (K / 32) * sizeof(float), s>>>(W, K, G, S, sc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    vq_sample_k<DT><<<dim3((L.ns + kQT - 1) / kQT, nblk), kQT, 0, s>>>(
        W, M, K, G, R, sample, L.ns, seed, sc, pts, cent, Cb, acc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const dim3 ga((L.ns + kQT * kPPT - 1) / (kQT * kPPT), nblk);
    for (uint32_t it = 0; it < iters; ++it) {
        vq_km_assign_k<<<ga, kQT, 0, s>>>(pts, L.ns, M, K, R, sample, cent, acc);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        vq_km_update_k<<<nblk, kCB, 0, s>>>(acc, cent, Cb);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const dim3 gf(M, (K / 2 + kQT * kPPT - 1) / (kQT * kPPT));
    vq_assign_k<DT><<<gf, kQT, 0, s>>>(W, K, G, R, sc, cent, IDX);
    return hipGetLastError();
}

}  // namespace

size_t vq_quant_ws_bytes(uint32_t M, uint32_t K, uint32_t scale_group, uint32_t rows_per_cb,
                         uint32_t sample) {
    return qws_layout(M, K, scale_group, rows_per_cb, sample).total;
}

uint32_t vq_quant_launches(uint32_t iters) { return 3 + 2 * iters; }

hipError_t launch_vq_quantize(const void* W, int w_dtype, uint32_t M, uint32_t K,
                              uint32_t rows_per_cb, uint32_t scale_group, uint32_t iters,
                              uint32_t sample, uint64_t seed, uint8_t* IDX, uint16_t* Cb,
                              uint16_t* S, void* ws, hipStream_t s) {
    uint8_t* w = reinterpret_cast<uint8_t*>(ws);
    if (w_dtype == KQ_F32)
        return vq_quant_go<KQ_F32>(W, M, K, scale_group, rows_per_cb, iters, sample, seed, IDX, Cb,
                                   S, w, s);
    if (w_dtype == KQ_BF16)
        return vq_quant_go<KQ_BF16>(W, M, K, scale_group, rows_per_cb, iters, sample, seed, IDX,
                                    Cb, S, w, s);
    return vq_quant_go<KQ_F16>(W, M, K, scale_group, rows_per_cb, iters, sample, seed, IDX, Cb, S,
                               w, s);
}

}  // namespace kq
