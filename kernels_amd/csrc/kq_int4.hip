// kq_int4.hip -- int4 group-affine GEMV, vector-ALU path (gfx950).
//
// Math (reference: int4-gemv/src/kernels.metal:17-31,397-448):
//   y[b,m] = sum_g S[m,g] * (sum_{k in g} q[m,k] x[b,k]) + B[m,g] * (sum_{k in g} x[b,k])
// evaluated per 32-weight chunk so the bias term lands exactly once per chunk.
//
// Mapping on CDNA4 (a decode GEMV is one streaming read of W; everything here
// serves keeping HBM requests in flight):
//   * persistent grid: one 1024-thread workgroup (16 waves) per CU; a wave
//     walks groups of R consecutive rows with a grid-wide stride, and each
//     row group as segments of S 64-chunk steps ("items"), so x is staged
//     once per CU and registers stay bounded for any K;
//   * a wave issues the 16-byte loads of its first item BEFORE the workgroup
//     stages x, and the next item's loads before computing the current one
//     (register double buffering), so the first HBM round trip overlaps the
//     staging and later ones overlap the math;
//   * x is staged in LDS as permuted fp16 pairs ([token][word%4][chunk], 16 B
//     per word: lane-consecutive chunks are conflict-free ds_read_b128) plus
//     per-chunk (sum, offset constant) -- this replaces the reference's
//     separate xsum32 launch; all staging loads of a thread are issued first;
//   * lane l owns chunk l + 64 s (s < S) of each row: a wave instruction reads
//     1 KiB of a row; nibbles become fp16 by AND-OR into fp16 exponents
//     (kq_device.h) and meet x in v_dot2_f32_f16 (fp32 accumulation); the
//     group metadata is applied once per chunk: acc += s*(d - xc) + b*xs;
//   * rows reduce with a wave64 butterfly; lane 0 stores y.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kMaxThreads = 1024;
constexpr int kStageRound = 2;  // x words per thread per staging round

template <bool BF>
__device__ __forceinline__ float meta_f(uint32_t v) {
    if constexpr (BF) return bf2f((uint16_t)v);
    else return h2f((uint16_t)v);
}

// Staging of NB activation vectors into LDS, in two phases so the x loads
// can be issued before the weight loads: the memory counter (vmcnt) retires
// in order, so x must be ahead of W in the queue or staging would wait for
// the first weight round trip.
template <int NB>
__device__ __forceinline__ void stage_x_load(const uint16_t* __restrict__ X, uint32_t K,
                                             uint32_t w0, u32x4 (&v)[kStageRound]) {
    const uint32_t nw = K >> 3, total = NB * nw, nthr = blockDim.x;
#pragma unroll
    for (int q = 0; q < kStageRound; ++q) {
        const uint32_t w = w0 + q * nthr + threadIdx.x;
        v[q] = u32x4{0, 0, 0, 0};
        if (w < total) {
            const uint32_t t = w / nw, wi = w - t * nw;
            v[q] = *reinterpret_cast<const u32x4*>(X + (size_t)t * K + (size_t)wi * 8);
        }
    }
}

template <int NB>
__device__ __forceinline__ void stage_x_store(uint32_t K, uint32_t w0,
                                              const u32x4 (&v)[kStageRound], u32x4* xp,
                                              float2* xk) {
    const uint32_t nch = K >> 5, nw = K >> 3, total = NB * nw, nthr = blockDim.x;
#pragma unroll
    for (int q = 0; q < kStageRound; ++q) {
        const uint32_t w = w0 + q * nthr + threadIdx.x;
        float s, c;
        word_consts(v[q], s, c);
        s = quad_sum(s);
        c = quad_sum(c);
        if (w < total) {
            const uint32_t t = w / nw, wi = w - t * nw;
            const uint32_t ch = wi >> 2, j = wi & 3;
            xp[(t * 4 + j) * nch + ch] = pair_perm(v[q]);
            if (j == 0) xk[t * nch + ch] = make_float2(s, c);
        }
    }
}

// Issue the loads of one item: rows rg*R .. rg*R+R-1, steps seg*S .. seg*S+S-1.
// SB: interleaved (scale, bias) dword per group; else separate S and B.
template <int S, int R, bool SB>
__device__ __forceinline__ void load_item(const uint32_t* __restrict__ W,
                                          const uint16_t* __restrict__ Sm,
                                          const uint16_t* __restrict__ Bm, uint32_t rg,
                                          uint32_t seg, uint32_t M, uint32_t nch, uint32_t gpr,
                                          uint32_t cshift, int lane, u32x4 (&w)[R][S],
                                          uint32_t (&m)[R][S]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t row = min(rg * R + r, M - 1);
        const u32x4* wrow = reinterpret_cast<const u32x4*>(W) + (size_t)row * nch;
        const uint32_t mrow = row * gpr;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const uint32_t c0 = 64u * (seg * S + s);
            if (c0 < nch) {  // wave-uniform
                const uint32_t c = c0 + 64 <= nch ? c0 + lane : min(c0 + lane, nch - 1);
                w[r][s] = ldg_nt(wrow + c);
                const uint32_t mi = mrow + (c >> cshift);
                if constexpr (SB)
                    m[r][s] = reinterpret_cast<const uint32_t*>(Sm)[mi];
                else
                    m[r][s] = (uint32_t)Sm[mi] | ((uint32_t)Bm[mi] << 16);
            }
        }
    }
}

template <int NB, int S, int R, bool BF>
__device__ __forceinline__ void compute_item(const u32x4 (&w)[R][S], const uint32_t (&m)[R][S],
                                             const u32x4* xp, const float2* xk, uint32_t nch,
                                             int lane, uint32_t seg, const DequantConsts& kc,
                                             float (&acc)[R][NB]) {
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const uint32_t c0 = 64u * (seg * S + s), c = c0 + lane;
        if (c0 < nch && c < nch) {
#pragma unroll
            for (int t = 0; t < NB; ++t) {
                const u32x4 p0 = xp[(t * 4 + 0) * nch + c];
                const u32x4 p1 = xp[(t * 4 + 1) * nch + c];
                const u32x4 p2 = xp[(t * 4 + 2) * nch + c];
                const u32x4 p3 = xp[(t * 4 + 3) * nch + c];
                const float2 k2 = xk[t * nch + c];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const u32x4 q = w[r][s];
                    float da = qdot8(q.x, p0, 0.0f, kc);
                    float db = qdot8(q.y, p1, 0.0f, kc);
                    da = qdot8(q.z, p2, da, kc);
                    db = qdot8(q.w, p3, db, kc);
                    const float sc = meta_f<BF>(m[r][s] & 0xFFFFu);
                    const float bi = meta_f<BF>(m[r][s] >> 16);
                    acc[r][t] = fmaf(sc, (da + db) - k2.y, fmaf(bi, k2.x, acc[r][t]));
                }
            }
        }
    }
}

// Wave-reduce a row group's accumulators, store y, reset the accumulators.
template <int NB, int R>
__device__ __forceinline__ void store_rows(float (&acc)[R][NB], int lane, uint32_t rg, uint32_t M,
                                           void* __restrict__ Y, int y_f32) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NB; ++t) {
            const float v = wave_sum(acc[r][t]);
            acc[r][t] = 0.0f;
            const uint32_t row = rg * R + r;
            if (lane == 0 && row < M) {
                const size_t o = (size_t)t * M + row;
                if (y_f32) reinterpret_cast<float*>(Y)[o] = v;
                else reinterpret_cast<uint16_t*>(Y)[o] = f2h(v);
            }
        }
}

// NB tokens; R rows per group; S 64-chunk steps per item (a row group is
// nseg = ceil(K/32/64/S) items). Items are double-buffered in registers.
template <int NB, int S, int R, bool SB, bool BF>
__global__ __launch_bounds__(kMaxThreads) void int4_gemv_valu(
    const uint32_t* __restrict__ W, const uint16_t* __restrict__ Sm,
    const uint16_t* __restrict__ Bm, const uint16_t* __restrict__ X, void* __restrict__ Y,
    int y_f32, uint32_t M, uint32_t K, uint32_t gshift) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nch = K >> 5;
    u32x4* xp = reinterpret_cast<u32x4*>(smem);                           // [NB][4][nch]
    float2* xk = reinterpret_cast<float2*>(smem + (size_t)NB * nch * 64);  // [NB][nch]
    const int lane = threadIdx.x & 63;
    const uint32_t nwaves = blockDim.x >> 6;
    const uint32_t stride = gridDim.x * nwaves;
    const uint32_t groups = (M + R - 1) / R;
    const uint32_t nseg = (((nch + 63) >> 6) + S - 1) / S;
    const uint32_t gpr = K >> gshift, cshift = gshift - 5;
    const uint32_t xwords = NB * (K >> 3), xround = blockDim.x * kStageRound;
    const DequantConsts kc;

    u32x4 wa[R][S], wb[R][S];
    uint32_t ma[R][S], mb[R][S];
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NB; ++t) acc[r][t] = 0.0f;

    // first staging round's x loads, then this wave's first item, then the
    // rest of the staging
    uint32_t rg = blockIdx.x * nwaves + (threadIdx.x >> 6), seg = 0;
    u32x4 xv[kStageRound];
    stage_x_load<NB>(X, K, 0, xv);
    if (rg < groups) load_item<S, R, SB>(W, Sm, Bm, rg, 0, M, nch, gpr, cshift, lane, wa, ma);
    stage_x_store<NB>(K, 0, xv, xp, xk);
    for (uint32_t w0 = xround; w0 < xwords; w0 += xround) {
        stage_x_load<NB>(X, K, w0, xv);
        stage_x_store<NB>(K, w0, xv, xp, xk);
    }
    __syncthreads();

    auto advance = [&](uint32_t& g, uint32_t& sg) {
        if (++sg == nseg) { sg = 0; g += stride; }
    };
    while (rg < groups) {
        uint32_t nrg = rg, nsg = seg;
        advance(nrg, nsg);
        if (nrg < groups)
            load_item<S, R, SB>(W, Sm, Bm, nrg, nsg, M, nch, gpr, cshift, lane, wb, mb);
        compute_item<NB, S, R, BF>(wa, ma, xp, xk, nch, lane, seg, kc, acc);
        if (seg == nseg - 1) store_rows<NB, R>(acc, lane, rg, M, Y, y_f32);
        rg = nrg;
        seg = nsg;
        if (rg >= groups) break;
        advance(nrg, nsg);
        if (nrg < groups)
            load_item<S, R, SB>(W, Sm, Bm, nrg, nsg, M, nch, gpr, cshift, lane, wa, ma);
        compute_item<NB, S, R, BF>(wb, mb, xp, xk, nch, lane, seg, kc, acc);
        if (seg == nseg - 1) store_rows<NB, R>(acc, lane, rg, M, Y, y_f32);
        rg = nrg;
        seg = nsg;
    }
}

int g_num_cu = 0;

int num_cu() {
    if (g_num_cu <= 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            g_num_cu = n;
        else
            g_num_cu = 256;
    }
    return g_num_cu;
}

template <int NB, int S, int R>
hipError_t launch3(const uint32_t* W, const uint16_t* Sm, const uint16_t* Bm, int bf16, bool sb,
                   const uint16_t* X, void* Y, bool y_f32, uint32_t M, uint32_t K,
                   uint32_t gshift, hipStream_t s) {
    const uint32_t groups = (M + R - 1) / R;
    const uint32_t waves = 16;
    uint32_t blocks = (groups + waves - 1) / waves;
    const uint32_t ncu = (uint32_t)num_cu();
    if (blocks > ncu) blocks = ncu;
    const size_t lds = (size_t)NB * (K >> 5) * 72;
    const int yf = y_f32 ? 1 : 0;
#define KQ_GO(SBV, BFV)                                                                        \
    int4_gemv_valu<NB, S, R, SBV, BFV><<<blocks, waves * 64, lds, s>>>(W, Sm, Bm, X, Y, yf, M, \
                                                                       K, gshift)
    if (sb && !bf16) KQ_GO(true, false);
    else if (!sb && !bf16) KQ_GO(false, false);
    else if (sb) KQ_GO(true, true);
    else KQ_GO(false, true);
#undef KQ_GO
    return hipGetLastError();
}

template <int NB>
hipError_t launch_nb(Int4Cfg cfg, const uint32_t* W, const uint16_t* Sm, const uint16_t* Bm,
                     int bf16, bool sb, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                     uint32_t K, uint32_t gshift, hipStream_t s) {
#define KQ_CASE(SS, RR)                                                                   \
    if (cfg.unroll == SS && cfg.rows == RR)                                               \
        return launch3<NB, SS, RR>(W, Sm, Bm, bf16, sb, X, Y, y_f32, M, K, gshift, s);
    if constexpr (NB == 1) {
        KQ_CASE(1, 1) KQ_CASE(1, 2) KQ_CASE(1, 4) KQ_CASE(2, 1) KQ_CASE(2, 2) KQ_CASE(4, 1)
    } else if constexpr (NB == 2) {
        KQ_CASE(1, 1) KQ_CASE(1, 2) KQ_CASE(2, 1) KQ_CASE(2, 2) KQ_CASE(4, 1)
    } else {
        KQ_CASE(1, 1) KQ_CASE(2, 1) KQ_CASE(4, 1)
    }
#undef KQ_CASE
    return hipErrorInvalidValue;
}

uint32_t log2u(uint32_t v) {
    uint32_t r = 0;
    while ((1u << r) < v) ++r;
    return r;
}

uint32_t steps_for(uint32_t K) { return ((K >> 5) + 63) / 64; }

}  // namespace

size_t int4_valu_lds_bytes(uint32_t K, uint32_t batch) { return (size_t)batch * (K >> 5) * 72; }

bool int4_valu_supported(uint32_t K, uint32_t batch, Int4Cfg cfg) {
    if (batch < 1 || batch > 16) return false;
    const int S = cfg.unroll, R = cfg.rows;
    const bool ok = (S == 1 && (R == 1 || R == 2 || R == 4)) || (S == 2 && (R == 1 || R == 2)) ||
                    (S == 4 && R == 1);
    return ok && int4_valu_lds_bytes(K, 1) <= 65536;
}

Int4Cfg int4_valu_default(uint32_t M, uint32_t K, uint32_t batch) {
    (void)M;
    const uint32_t st = steps_for(K);
    Int4Cfg c;
    c.unroll = st <= 1 ? 1 : st <= 2 ? 2 : 4;
    c.rows = c.unroll == 1 ? 4 : c.unroll == 2 ? 2 : 1;
    // more tokens per pass keep more x pairs live: hold rows*tokens <= 4
    const int nb = batch >= 4 ? 4 : batch >= 2 ? 2 : 1;
    while (c.rows > 1 && c.rows * nb > 4) c.rows /= 2;
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
        uint32_t nb = (left >= 4 && int4_valu_lds_bytes(K, 4) <= 65536) ? 4
                    : (left >= 2 && int4_valu_lds_bytes(K, 2) <= 65536) ? 2 : 1;
        while (nb > 1 && cfg.rows * (int)nb > 4) nb /= 2;  // register budget
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
