// kq_moe_unfused.hip -- the MoE decode block with one operation per launch,
// the way an eager framework runs it: every intermediate goes through device
// memory. It exists to make the launch-count comparison with the
// three-launch block a measurement: the unfused reference path of
// moe-fused/src/kernels.metal:267-397, dispatched by encodeUnfused
// moe-fused/src/main.mm:208-284. The numerical contract is the block's.
//
// Launches (one token, top_k = k), in stream order:
//   router logits (the block's router kernel, its top-k tail off)   1
//   top-k by repeated argmax -> idx, the selected logits             1
//   softmax over the selected logits -> wgt                          1
//   per slot: gate GEMV, up GEMV, SwiGLU (+ output biases) -> H[s]   3k
//   per slot: down GEMV, weighted accumulate (+ output bias)         2k
// = 3 + 5k (23 at top-4). The reference's 28 add five x-sum passes (the
// per-chunk activation sums its GEMV reads); the GEMV here is the vector
// int4 GEMV of kq_int4.hip, which forms those sums while it stages x, and
// which reads the slot's expert index from idx on the device (no host round
// trip). The output biases are applied by each GEMV's consumer, in the same
// fp32 order as the fused kernels: swiglu(g + bi_g, u + bi_u) and
// acc + wgt * (v + bi_d).
#include "kq_internal.h"
#include "kq_moe_device.h"

namespace kq {

namespace {

constexpr uint32_t kUMaxTopK = 8;
constexpr uint32_t kUThreads = 256;

// Workspace of the unfused block (no initialisation needed: every buffer is
// written before it is read).
struct UWs {
    size_t lg, sel, g, u, v, acc, total;
};

UWs uws_layout(const kq_moe_desc& d) {
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    UWs L;
    L.lg = 0;
    L.sel = al(4ull * d.n_experts);
    L.g = L.sel + al(4ull * kUMaxTopK);
    L.u = L.g + al(4ull * d.inter);
    L.v = L.u + al(4ull * d.inter);
    L.acc = L.v + al(4ull * d.hidden);
    L.total = L.acc + al(4ull * d.hidden);
    return L;
}

// Top-k by repeated argmax (u_topk, moe-fused/src/kernels.metal:310-320): pass
// j picks the largest remaining logit, strictly greater wins so ties go to
// the lowest index, and the winner is removed. NaN and -inf are never
// selectable; a pass with nothing selectable yields index 0 and -inf, as the
// block's router does (the same topk_select). One wave, up to 4 logits per
// lane; slot j is written by lane j.
__global__ __launch_bounds__(64) void u_topk_k(const float* __restrict__ lg, uint32_t NE,
                                               uint32_t TK, uint32_t* __restrict__ idx,
                                               float* __restrict__ sel) {
    const uint32_t lane = threadIdx.x;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t ei = lane + 64 * q;
        v[q] = cand(lg[min(ei, NE - 1)], ei < NE);
    }
    float chosen[kUMaxTopK];
    uint32_t pick[kUMaxTopK];
    topk_select(v, TK, pick, chosen);
#pragma unroll
    for (uint32_t j = 0; j < kUMaxTopK; ++j) {
        if (j < TK && lane == j) {
            idx[j] = pick[j];
            sel[j] = chosen[j];
        }
    }
}

// Softmax over the k selected logits (u_softmax_k,
// moe-fused/src/kernels.metal:322-331): max, exp(l - max), summed in slot
// order, divided -- the arithmetic of the block's router tail.
__global__ __launch_bounds__(64) void u_softmax_k(const float* __restrict__ sel, uint32_t TK,
                                                  float* __restrict__ wgt) {
    if (threadIdx.x != 0) return;
    float mx = sel[0];
#pragma unroll
    for (uint32_t j = 1; j < kUMaxTopK; ++j)
        if (j < TK) mx = fmaxf(mx, sel[j]);
    float ex[kUMaxTopK], sum = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kUMaxTopK; ++j) {
        ex[j] = 0.0f;
        if (j < TK) {
            ex[j] = expf(sel[j] - mx);
            sum += ex[j];
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < kUMaxTopK; ++j)
        if (j < TK) wgt[j] = ex[j] / sum;
}

// H[i] = half(swiglu(g[i] + BIg[i], u[i] + BIu[i])) for the slot's expert
// (u_swiglu, moe-fused/src/kernels.metal:373-381, with the GEMV's output
// bias of moe-fused/src/kernels.metal:365-368).
__global__ __launch_bounds__(kUThreads) void u_swiglu_k(const float* __restrict__ g,
                                                        const float* __restrict__ u,
                                                        const uint8_t* __restrict__ pool,
                                                        uint64_t blob, uint64_t bi_gate,
                                                        uint64_t bi_up, const uint32_t* sel_e,
                                                        uint16_t* __restrict__ h, uint32_t n) {
    const uint32_t i = blockIdx.x * kUThreads + threadIdx.x;
    if (i >= n) return;
    const uint8_t* base = pool + (size_t)__builtin_amdgcn_readfirstlane(*sel_e) * blob;
    const float bg = bf2f(reinterpret_cast<const uint16_t*>(base + bi_gate)[i]);
    const float bu = bf2f(reinterpret_cast<const uint16_t*>(base + bi_up)[i]);
    h[i] = f2h(swiglu(g[i] + bg, u[i] + bu));
}

// acc[i] = (slot 0 ? 0 : acc[i]) + wgt[s] * (v[i] + BId[i]); the last slot
// writes Y instead (u_axpy, moe-fused/src/kernels.metal:383-392). The slots
// are summed in k order, as the block's combine does.
__global__ __launch_bounds__(kUThreads) void u_axpy_k(const float* __restrict__ v,
                                                      const uint8_t* __restrict__ pool,
                                                      uint64_t blob, uint64_t bi_down,
                                                      const uint32_t* sel_e,
                                                      const float* __restrict__ wgt, uint32_t s,
                                                      float* __restrict__ acc, void* Y,
                                                      uint32_t y_f32, uint32_t last, uint32_t n) {
    const uint32_t i = blockIdx.x * kUThreads + threadIdx.x;
    if (i >= n) return;
    const uint8_t* base = pool + (size_t)__builtin_amdgcn_readfirstlane(*sel_e) * blob;
    const float b = bf2f(reinterpret_cast<const uint16_t*>(base + bi_down)[i]);
    const float a = (s == 0 ? 0.0f : acc[i]) + wgt[s] * (v[i] + b);
    if (!last) acc[i] = a;
    else if (y_f32) reinterpret_cast<float*>(Y)[i] = a;
    else reinterpret_cast<uint16_t*>(Y)[i] = f2h(a);
}

}  // namespace

size_t moe_unfused_ws_bytes(const kq_moe_desc& d) { return uws_layout(d).total; }

uint32_t moe_unfused_launches(const kq_moe_desc& d) { return 3 + 5 * d.top_k; }

hipError_t launch_moe_unfused(const uint8_t* pool, const kq_moe_desc& d, const void* R, bool r_f32,
                              const void* X, bool x_f32, uint32_t* idx, float* wgt, uint16_t* xh,
                              uint16_t* H, void* Y, bool y_f32, void* ws, hipStream_t s) {
    const UWs L = uws_layout(d);
    uint8_t* w = reinterpret_cast<uint8_t*>(ws);
    float* lg = reinterpret_cast<float*>(w + L.lg);
    float* sel = reinterpret_cast<float*>(w + L.sel);
    float* G = reinterpret_cast<float*>(w + L.g);
    float* U = reinterpret_cast<float*>(w + L.u);
    float* V = reinterpret_cast<float*>(w + L.v);
    float* acc = reinterpret_cast<float*>(w + L.acc);
    const uint16_t* x = x_f32 ? xh : reinterpret_cast<const uint16_t*>(X);
    const Int4Cfg auto_cfg{0, 0};
    hipError_t e;

    if ((e = launch_moe_logits(R, r_f32, X, x_f32, 1, d, xh, lg, s)) != hipSuccess) return e;
    u_topk_k<<<1, 64, 0, s>>>(lg, d.n_experts, d.top_k, idx, sel);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    u_softmax_k<<<1, 64, 0, s>>>(sel, d.top_k, wgt);
    if ((e = hipGetLastError()) != hipSuccess) return e;

    // one projection of expert idx[slot]: W, S, B of expert 0, moved on the device
    auto proj = [&](uint64_t off, const uint16_t* xin, float* yout, uint32_t M, uint32_t K,
                    uint32_t slot) {
        const uint8_t* p = pool + off;
        return launch_int4_valu(reinterpret_cast<const uint32_t*>(p + d.sub_w),
                                reinterpret_cast<const uint16_t*>(p + d.sub_s),
                                reinterpret_cast<const uint16_t*>(p + d.sub_b), 1, false, xin,
                                yout, true, M, K, 64, 1, auto_cfg, s, idx + slot, d.blob);
    };
    const uint32_t gi = (d.inter + kUThreads - 1) / kUThreads;
    const uint32_t gh = (d.hidden + kUThreads - 1) / kUThreads;
    for (uint32_t k = 0; k < d.top_k; ++k) {
        if ((e = proj(d.off_gate, x, G, d.inter, d.hidden, k)) != hipSuccess) return e;
        if ((e = proj(d.off_up, x, U, d.inter, d.hidden, k)) != hipSuccess) return e;
        u_swiglu_k<<<gi, kUThreads, 0, s>>>(G, U, pool, d.blob, d.off_gate + d.sub_bi,
                                            d.off_up + d.sub_bi, idx + k,
                                            H + (size_t)k * d.inter, d.inter);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    for (uint32_t k = 0; k < d.top_k; ++k) {
        if ((e = proj(d.off_down, H + (size_t)k * d.inter, V, d.hidden, d.inter, k)) != hipSuccess)
            return e;
        u_axpy_k<<<gh, kUThreads, 0, s>>>(V, pool, d.blob, d.off_down + d.sub_bi, idx + k, wgt, k,
                                          acc, Y, y_f32 ? 1 : 0, k + 1 == d.top_k ? 1 : 0,
                                          d.hidden);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace kq
