// kq_vq.hip -- codebook (VQ d=2, 256 entries) dequant-GEMV (gfx950).
//
// Format (reference vq-gemv/src/kernels.metal:15-27, generalised):
//   w[m, 2i+t] = S[m, 2i/scale_group] * C[m/rows_per_cb][IDX[m,i]][t]
// No bias and so no sum-of-x term (the codebook absorbs the group mean).
//
// Mapping on CDNA4:
//   * the workgroup stages x (natural fp16 pairs, [token][word%4][chunk]
//     layout for conflict-free ds_read_b128) and the codebook block(s) its
//     rows need (256 x half2 = 1 KiB each) into LDS;
//   * each wave owns R rows; lane l loads 16 indices (32 weights, one 16-byte
//     global load) per 64-chunk step, U steps in flight;
//   * each index byte addresses one half2 codeword in LDS (ds_read_b32), which
//     is dotted with its activation pair by v_dot2_f32_f16 (fp32 accumulate);
//   * the row scale applies once per 32-weight chunk (scale_group % 32 == 0).
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;

template <int NB, int R, int U>
__global__ __launch_bounds__(kThreads) void vq_gemv_k(
    const uint8_t* __restrict__ IDX, const uint16_t* __restrict__ C,
    const uint16_t* __restrict__ S, const uint16_t* __restrict__ X, void* __restrict__ Y,
    int y_f32, uint32_t M, uint32_t K, uint32_t rpc, uint32_t sg_shift) {
    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t nch = K >> 5, nw = K >> 3;
    u32x4* xq = reinterpret_cast<u32x4*>(smem);                         // [NB][4][nch]
    uint32_t* cb = reinterpret_cast<uint32_t*>(smem + (size_t)NB * nch * 64);  // [ncb][256]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t rows_per_block = kWaves * R;
    const uint32_t mfirst = blockIdx.x * rows_per_block;
    const uint32_t mlast = min(mfirst + rows_per_block, M) - 1;
    const uint32_t cb0 = mfirst / rpc, ncb = mlast / rpc - cb0 + 1;

    for (uint32_t w = tid; w < NB * nw; w += kThreads) {
        const uint32_t t = w / nw, wi = w - t * nw;
        xq[(t * 4 + (wi & 3)) * nch + (wi >> 2)] =
            *reinterpret_cast<const u32x4*>(X + (size_t)t * K + (size_t)wi * 8);
    }
    for (uint32_t i = tid; i < ncb * 256; i += kThreads)
        cb[i] = reinterpret_cast<const uint32_t*>(C)[(size_t)cb0 * 256 + i];
    __syncthreads();

    const uint32_t row0 = mfirst + wave * R;
    if (row0 >= M) return;
    // sg_shift == 0 encodes one scale per row (scale_group == K)
    const uint32_t spr = sg_shift ? K >> sg_shift : 1;   // scales per row
    const uint32_t cshift = sg_shift ? sg_shift - 5 : 31; // chunk -> scale index

    const u32x4* irow[R];
    const uint16_t* srow[R];
    const uint32_t* crow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint32_t m = min(row0 + r, M - 1);
        irow[r] = reinterpret_cast<const u32x4*>(IDX + (size_t)m * (K >> 1));
        srow[r] = S + (size_t)m * spr;
        crow[r] = cb + (m / rpc - cb0) * 256;
    }
    float acc[R][NB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < NB; ++t) acc[r][t] = 0.0f;

    for (uint32_t it = 0; it < nch; it += 64 * U) {
        u32x4 iv[U][R];
        float sc[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (it + 64 * u < nch) {
                const uint32_t c = min(it + 64 * u + lane, nch - 1);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    iv[u][r] = ldg_nt(irow[r] + c);
                    sc[u][r] = h2f(srow[r][sg_shift ? (c >> cshift) : 0]);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t c = it + 64 * u + lane;
            if (it + 64 * u < nch && c < nch) {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    // 16 codewords of this chunk, looked up once, reused per token
                    uint32_t cw[16];
                    const u32x4 v = iv[u][r];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const uint32_t word = q == 0 ? v.x : q == 1 ? v.y : q == 2 ? v.z : v.w;
                        cw[4 * q + 0] = crow[r][word & 0xFF];
                        cw[4 * q + 1] = crow[r][(word >> 8) & 0xFF];
                        cw[4 * q + 2] = crow[r][(word >> 16) & 0xFF];
                        cw[4 * q + 3] = crow[r][word >> 24];
                    }
#pragma unroll
                    for (int t = 0; t < NB; ++t) {
                        float da = 0.0f, db = 0.0f;
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const u32x4 xv = xq[(t * 4 + q) * nch + c];  // x[32c+8q .. +7]
                            da = dot2(cw[4 * q + 0], xv.x, da);
                            db = dot2(cw[4 * q + 1], xv.y, db);
                            da = dot2(cw[4 * q + 2], xv.z, da);
                            db = dot2(cw[4 * q + 3], xv.w, db);
                        }
                        acc[r][t] = fmaf(sc[u][r], da + db, acc[r][t]);
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
hipError_t vq_launch3(const uint8_t* IDX, const uint16_t* C, const uint16_t* S, const uint16_t* X,
                      void* Y, bool y_f32, uint32_t M, uint32_t K, uint32_t rpc, uint32_t sgs,
                      hipStream_t s) {
    const uint32_t rpb = kWaves * R;
    const uint32_t ncb_max = (rpb - 1) / rpc + 2;
    const size_t lds = (size_t)NB * (K >> 5) * 64 + (size_t)ncb_max * 1024;
    const dim3 grid((M + rpb - 1) / rpb);
    vq_gemv_k<NB, R, U><<<grid, kThreads, lds, s>>>(IDX, C, S, X, Y, y_f32 ? 1 : 0, M, K, rpc, sgs);
    return hipGetLastError();
}

template <int NB, int R>
hipError_t vq_launch2(int U, const uint8_t* IDX, const uint16_t* C, const uint16_t* S,
                      const uint16_t* X, void* Y, bool y_f32, uint32_t M, uint32_t K, uint32_t rpc,
                      uint32_t sgs, hipStream_t s) {
    switch (U) {
        case 1: return vq_launch3<NB, R, 1>(IDX, C, S, X, Y, y_f32, M, K, rpc, sgs, s);
        case 2: return vq_launch3<NB, R, 2>(IDX, C, S, X, Y, y_f32, M, K, rpc, sgs, s);
        case 4: return vq_launch3<NB, R, 4>(IDX, C, S, X, Y, y_f32, M, K, rpc, sgs, s);
        default: return vq_launch3<NB, R, 8>(IDX, C, S, X, Y, y_f32, M, K, rpc, sgs, s);
    }
}

}  // namespace

size_t vq_lds_bytes(uint32_t K, uint32_t nb) { return (size_t)nb * (K >> 5) * 64 + 6 * 1024; }

hipError_t launch_vq(const uint8_t* IDX, const uint16_t* C, const uint16_t* S, const uint16_t* X,
                     void* Y, bool y_f32, uint32_t M, uint32_t K, uint32_t rows_per_cb,
                     uint32_t scale_group, uint32_t batch, hipStream_t s) {
    uint32_t sgs = 0;  // 0: one scale per row
    if (scale_group != K)
        while ((1u << sgs) < scale_group) ++sgs;
    const uint32_t steps = ((K >> 5) + 63) / 64;
    const int U = steps <= 1 ? 1 : steps <= 2 ? 2 : steps <= 4 ? 4 : 8;
    const size_t ysz = y_f32 ? 4 : 2;
    // tokens in groups of 4, 2, 1 (each group one launch over the same rows)
    for (uint32_t t0 = 0; t0 < batch;) {
        const uint32_t left = batch - t0;
        const uint32_t nb = left >= 4 && vq_lds_bytes(K, 4) <= 65536 ? 4 : left >= 2 ? 2 : 1;
        const uint16_t* Xt = X + (size_t)t0 * K;
        void* Yt = reinterpret_cast<uint8_t*>(Y) + (size_t)t0 * M * ysz;
        hipError_t e;
        if (nb == 4) e = vq_launch2<4, 1>(U, IDX, C, S, Xt, Yt, y_f32, M, K, rows_per_cb, sgs, s);
        else if (nb == 2) e = vq_launch2<2, 1>(U, IDX, C, S, Xt, Yt, y_f32, M, K, rows_per_cb, sgs, s);
        else e = vq_launch2<1, 1>(U, IDX, C, S, Xt, Yt, y_f32, M, K, rows_per_cb, sgs, s);
        if (e != hipSuccess) return e;
        t0 += nb;
    }
    return hipSuccess;
}

}  // namespace kq
