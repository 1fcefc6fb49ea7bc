// kq_moe.hip -- the MoE decode block (gfx950).
//
// Reference: moe-fused/src/kernels.metal:98-265 (router_topk,
// fused_gate_up_swiglu, fused_down_combine) and the block reference
// moe-fused/src/main.mm:302-334. The block has two grid-wide dependencies
// (the selected experts before the gather; all of h before down). On CDNA4
// an in-kernel cross-workgroup handshake needs an agent-scope release, which
// writes back the XCD's L2 -- far too slow for a few-microsecond block -- so
// every dependency here is a kernel boundary and nothing inside a kernel
// waits on another workgroup:
//
// 1. moe_logits_k: router logits, one wave per expert reading its router row
//    once for all tokens (fp32 accumulate), to the workspace; also half(x)
//    when x is fp32 (router_topk writes xh the same way).
// 2. moe_select_k (standalone router only): top-k + softmax per token.
// 3. moe_gate_up_k: grid (16-row tile, u). Each workgroup derives the
//    ascending list of distinct selected experts, takes the u-th and reads
//    its gate/up rows once for every token slot that chose it. In the fused
//    block each workgroup first runs top-k itself from the logits (a few
//    hundred instructions, cheaper than a launch); workgroup (0,0) publishes
//    idx/wgt. A half-wave (32 lanes) owns a gate row, the other half the
//    matching up row (K = 2880 = 90 chunks -> 3 per lane), so SwiGLU happens
//    on the two half-wave sums.
// 4. moe_down_k: grid (8-row tile). A workgroup covers its rows for all
//    selected experts (one wave per expert, looping), keeps per-slot
//    wgt*(down.h + bias) in LDS and sums them in slot order: deterministic,
//    no atomics.
//
// The activation a wave multiplies (x or h, per token slot) sits in its
// registers as permuted fp16 pairs for all of the wave's rows; the weights
// are dequantised with the AND-OR trick of kq_device.h; bf16 group scale and
// bias apply once per 32-weight chunk.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kThreads = 256;
constexpr int kGuRows = 16;   // gate/up rows per workgroup (4 waves x 4 rows)
constexpr int kGuRW = 4;      // gate/up rows per wave
constexpr int kDnRows = 8;    // down rows per workgroup
constexpr int kMaxSlots = 128;
constexpr int kMaxTopK = 8;

struct WsLayout {
    size_t lg, total;
};

WsLayout ws_layout(const kq_moe_desc& d, uint32_t batch) {
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    WsLayout L;
    L.lg = 0;
    L.total = al(L.lg + 4ull * batch * d.n_experts);
    return L;
}

// ---------------------------------------------------------------------------
// 1. router logits
// ---------------------------------------------------------------------------
template <bool F32>
__device__ __forceinline__ void load8(const void* p, size_t i, float v[8]) {
    if constexpr (F32) {
        const f32x4* q = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + i);
        const f32x4 a = q[0], b = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
        const u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(p) + i);
        v[0] = h2f(a.x & 0xFFFF); v[1] = h2f(a.x >> 16); v[2] = h2f(a.y & 0xFFFF); v[3] = h2f(a.y >> 16);
        v[4] = h2f(a.z & 0xFFFF); v[5] = h2f(a.z >> 16); v[6] = h2f(a.w & 0xFFFF); v[7] = h2f(a.w >> 16);
    }
}

template <bool RF32, bool XF32>
__global__ __launch_bounds__(kThreads) void moe_logits_k(const void* __restrict__ R,
                                                         const void* __restrict__ X,
                                                         uint32_t batch, uint32_t NE,
                                                         uint32_t HID, uint16_t* __restrict__ xh,
                                                         float* __restrict__ lg) {
    constexpr int NBMAX = 16;
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t e = blockIdx.x * (kThreads / 64) + (tid >> 6);

    if (XF32 && xh) {  // fp16 copy of x for the projections
        const uint32_t tot = batch * HID;
        for (uint32_t i = blockIdx.x * kThreads + tid; i < tot; i += gridDim.x * kThreads)
            xh[i] = f2h(reinterpret_cast<const float*>(X)[i]);
    }
    if (e >= NE) return;
    float acc[NBMAX];
#pragma unroll
    for (int t = 0; t < NBMAX; ++t) acc[t] = 0.0f;
    for (uint32_t k = lane * 8; k < HID; k += 64 * 8) {
        float r[8];
        load8<RF32>(R, (size_t)e * HID + k, r);
#pragma unroll
        for (int t = 0; t < NBMAX; ++t) {
            if ((uint32_t)t < batch) {
                float x[8];
                load8<XF32>(X, (size_t)t * HID + k, x);
                float a = acc[t];
#pragma unroll
                for (int i = 0; i < 8; ++i) a = fmaf(r[i], x[i], a);
                acc[t] = a;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NBMAX; ++t) {
        if ((uint32_t)t < batch) {
            const float v = wave_sum(acc[t]);
            if (lane == 0) lg[(size_t)t * NE + e] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// top-k + softmax of one token, one wave (moe-fused/src/kernels.metal:149-162):
// k passes of "strictly greater wins, ascending scan" -- ties go to the
// lowest index, NaN and -inf are never selectable, and a pass with nothing
// selectable picks expert 0 -- then softmax over the chosen logits.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool better(float va, uint32_t ia, float vb, uint32_t ib) {
    const bool oka = va > -INFINITY, okb = vb > -INFINITY;
    if (oka != okb) return oka;
    if (!oka) return ia < ib;
    return va > vb || (va == vb && ia < ib);
}

__device__ void topk_wave(const float* __restrict__ L, uint32_t NE, uint32_t TK,
                          uint32_t* idx_out, float* wgt_out) {
    const uint32_t lane = threadIdx.x & 63;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t ei = lane + 64 * q;
        v[q] = ei < NE ? L[ei] : -INFINITY;
    }
    float chosen[kMaxTopK];
    uint32_t pick[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        chosen[j] = -INFINITY;
        pick[j] = 0;
        if ((uint32_t)j < TK) {
            float bv = -INFINITY;
            uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t ei = lane + 64 * q;
                if (ei < NE && better(v[q], ei, bv, bi)) { bv = v[q]; bi = ei; }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o, 64);
                const uint32_t oi = __shfl_xor(bi, o, 64);
                if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
            }
            if (!(bv > -INFINITY)) { bv = -INFINITY; bi = 0; }
            chosen[j] = bv;
            pick[j] = bi;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (lane + 64 * q == bi) v[q] = -INFINITY;
        }
    }
    if (lane == 0) {
        float mx = chosen[0];
#pragma unroll
        for (int j = 1; j < kMaxTopK; ++j)
            if ((uint32_t)j < TK) mx = fmaxf(mx, chosen[j]);
        float ex[kMaxTopK], sum = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j) {
            ex[j] = 0.0f;
            if ((uint32_t)j < TK) { ex[j] = expf(chosen[j] - mx); sum += ex[j]; }
        }
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if ((uint32_t)j < TK) { idx_out[j] = pick[j]; wgt_out[j] = ex[j] / sum; }
    }
}

__global__ __launch_bounds__(kThreads) void moe_select_k(const float* __restrict__ lg,
                                                         uint32_t batch, uint32_t NE,
                                                         uint32_t TK, uint32_t* __restrict__ idx,
                                                         float* __restrict__ wgt) {
    for (uint32_t t = threadIdx.x >> 6; t < batch; t += kThreads / 64)
        topk_wave(lg + (size_t)t * NE, NE, TK, idx + t * TK, wgt + t * TK);
}

// ---------------------------------------------------------------------------
// Which expert a work item handles, and its token slots
// ---------------------------------------------------------------------------
// Marks the experts selected by the slots in an LDS bitmap of 8 words.
__device__ __forceinline__ void mark_experts(const uint32_t* idx, uint32_t nslots, uint32_t NE,
                                             uint32_t* bits) {
    const int tid = threadIdx.x;
    if (tid < 8) bits[tid] = 0;
    __syncthreads();
    if ((uint32_t)tid < nslots) {
        const uint32_t e = min(idx[tid], NE - 1);
        atomicOr(&bits[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
}

struct Plan {
    uint32_t e;         // expert id (valid if u < n_unique)
    uint32_t n_unique;  // distinct experts selected
    uint64_t m0, m1;    // slots s (s < 64: bit s of m0; else bit s-64 of m1)
};

// The u-th smallest marked expert and the slots that selected it (wave-level;
// every lane of the wave must be active).
__device__ Plan plan_for(const uint32_t* idx, uint32_t nslots, uint32_t NE, uint32_t u,
                         const uint32_t* bits) {
    const uint32_t lane = threadIdx.x & 63;
    Plan p;
    p.e = 0xFFFFFFFFu;
    uint32_t cnt = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t b = bits[w];
        const uint32_t pc = __popc(b);
        if (p.e == 0xFFFFFFFFu && u < cnt + pc) {
            for (uint32_t i = 0; i < u - cnt; ++i) b &= b - 1;
            p.e = w * 32 + __builtin_ctz(b);
        }
        cnt += pc;
    }
    p.n_unique = cnt;
    const bool q0 = lane < nslots && min(idx[lane], NE - 1) == p.e;
    const bool q1 = lane + 64 < nslots && min(idx[lane + 64], NE - 1) == p.e;
    p.m0 = __ballot(q0);
    p.m1 = __ballot(q1);
    return p;
}

__device__ __forceinline__ uint32_t pop_slot(uint64_t& m0, uint64_t& m1) {
    if (m0) { const uint32_t s = __builtin_ctzll(m0); m0 &= m0 - 1; return s; }
    const uint32_t s = 64 + __builtin_ctzll(m1);
    m1 &= m1 - 1;
    return s;
}

// ---------------------------------------------------------------------------
// register-resident activation: chunks c0 + 32j (j < J) of one fp16 vector
// ---------------------------------------------------------------------------
template <int J>
struct Act {
    u32x4 p[J][4];   // permuted pairs of the chunk's 4 words
    float xs[J];     // chunk sum
    float xc[J];     // chunk offset constant
};

template <int J>
__device__ __forceinline__ void act_load(const uint16_t* __restrict__ v, uint32_t nch, uint32_t c0,
                                         u32x4 (&raw)[J][4]) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t c = min(c0 + 32 * j, nch - 1);
        const u32x4* src = reinterpret_cast<const u32x4*>(v) + (size_t)c * 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) raw[j][q] = src[q];
    }
}

template <int J>
__device__ __forceinline__ void act_prep(const u32x4 (&raw)[J][4], Act<J>& a) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float s = 0.0f, c = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float ws, wc;
            word_consts(raw[j][q], ws, wc);
            s += ws;
            c += wc;
            a.p[j][q] = pair_perm(raw[j][q]);
        }
        a.xs[j] = s;
        a.xc[j] = c;
    }
}

// Load J chunks (lane c0 + 32j) of row m of a projection plus bf16 S|B.
template <int J>
__device__ __forceinline__ void load_row(const uint8_t* proj, const kq_moe_desc& d, uint32_t K,
                                         uint32_t m, uint32_t c0, u32x4 (&w)[J],
                                         uint32_t (&mt)[J]) {
    const uint32_t nch = K >> 5, gpr = K >> 6;
    const u32x4* W = reinterpret_cast<const u32x4*>(proj + d.sub_w) + (size_t)m * nch;
    const uint16_t* S = reinterpret_cast<const uint16_t*>(proj + d.sub_s) + (size_t)m * gpr;
    const uint16_t* B = reinterpret_cast<const uint16_t*>(proj + d.sub_b) + (size_t)m * gpr;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t c = min(c0 + 32 * j, nch - 1);
        w[j] = ldg_nt(W + c);
        mt[j] = (uint32_t)S[c >> 1] | ((uint32_t)B[c >> 1] << 16);
    }
}

// Per-lane partial dot of one row's J chunks with a register activation.
template <int J>
__device__ __forceinline__ float row_dot(const u32x4 (&w)[J], const uint32_t (&mt)[J],
                                         const Act<J>& a, uint32_t nch, uint32_t c0,
                                         const DequantConsts& kc) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (c0 + 32 * j < nch) {
            float da = qdot8(w[j].x, a.p[j][0], 0.0f, kc);
            float db = qdot8(w[j].y, a.p[j][1], 0.0f, kc);
            da = qdot8(w[j].z, a.p[j][2], da, kc);
            db = qdot8(w[j].w, a.p[j][3], db, kc);
            const float s = bf2f(mt[j] & 0xFFFFu), b = bf2f(mt[j] >> 16);
            acc = fmaf(s, (da + db) - a.xc[j], fmaf(b, a.xs[j], acc));
        }
    }
    return acc;
}

// ---------------------------------------------------------------------------
// 3. gather + gate + up + SwiGLU
// ---------------------------------------------------------------------------
template <int J, bool FROM_LOGITS>
__global__ __launch_bounds__(kThreads) void moe_gate_up_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx_g,
    float* __restrict__ wgt_pub, uint32_t* __restrict__ idx_pub, const float* __restrict__ lg,
    const uint16_t* __restrict__ xh, uint16_t* __restrict__ H, uint32_t batch) {
    __shared__ uint32_t bits[8];
    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    const uint32_t HID = d.hidden, IN = d.inter, TK = d.top_k;
    const uint32_t nslots = batch * TK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    const uint32_t* idx = idx_g;
    if constexpr (FROM_LOGITS) {
        for (uint32_t t = wave; t < batch; t += kThreads / 64)
            topk_wave(lg + (size_t)t * d.n_experts, d.n_experts, TK, s_idx + t * TK,
                      s_wgt + t * TK);
        __syncthreads();
        if (blockIdx.x == 0 && blockIdx.y == 0 && (uint32_t)tid < nslots) {
            idx_pub[tid] = s_idx[tid];  // for the down pass and the caller
            wgt_pub[tid] = s_wgt[tid];
        }
        idx = s_idx;
    }
    mark_experts(idx, nslots, d.n_experts, bits);
    const Plan p = plan_for(idx, nslots, d.n_experts, blockIdx.y, bits);
    if (blockIdx.y >= p.n_unique) return;

    const uint32_t half = lane >> 5, c0 = lane & 31, nch = HID >> 5;
    const uint8_t* blob = pool + (size_t)p.e * d.blob;
    const uint8_t* proj = blob + (half ? d.off_up : d.off_gate);
    const uint32_t m0 = blockIdx.x * kGuRows + wave * kGuRW;
    const DequantConsts kc;

    uint64_t sm0 = p.m0, sm1 = p.m1;
    uint32_t slot = pop_slot(sm0, sm1);
    // x of the first slot ahead of the weights in the memory queue
    u32x4 raw[J][4];
    act_load<J>(xh + (size_t)(slot / TK) * HID, nch, c0, raw);

    u32x4 w[kGuRW][J];
    uint32_t mt[kGuRW][J];
#pragma unroll
    for (int r = 0; r < kGuRW; ++r) load_row<J>(proj, d, HID, min(m0 + r, IN - 1), c0, w[r], mt[r]);
    float bg = 0.0f, bu = 0.0f;
    if (lane < kGuRW && m0 + lane < IN) {
        bg = bf2f(reinterpret_cast<const uint16_t*>(blob + d.off_gate + d.sub_bi)[m0 + lane]);
        bu = bf2f(reinterpret_cast<const uint16_t*>(blob + d.off_up + d.sub_bi)[m0 + lane]);
    }

    while (true) {
        Act<J> a;
        act_prep<J>(raw, a);
        float g[kGuRW], u[kGuRW];
#pragma unroll
        for (int r = 0; r < kGuRW; ++r) {
            const float2 hs = half_sums(row_dot<J>(w[r], mt[r], a, nch, c0, kc));
            g[r] = hs.x;
            u[r] = hs.y;
        }
#pragma unroll
        for (int r = 0; r < kGuRW; ++r) {
            if (lane == r && m0 + r < IN) {
                const float gg = fminf(g[r] + bg, 7.0f);
                const float uu = fminf(fmaxf(u[r] + bu, -7.0f), 7.0f);
                const float h = (gg / (1.0f + expf(-1.702f * gg))) * (uu + 1.0f);
                H[(size_t)slot * IN + m0 + r] = f2h(h);
            }
        }
        if (!(sm0 | sm1)) break;
        slot = pop_slot(sm0, sm1);
        act_load<J>(xh + (size_t)(slot / TK) * HID, nch, c0, raw);
    }
}

// ---------------------------------------------------------------------------
// 4. gather + down + weighted combine
// ---------------------------------------------------------------------------
template <int J>
__global__ __launch_bounds__(kThreads) void moe_down_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx,
    const float* __restrict__ wgt, const uint16_t* __restrict__ H, void* __restrict__ Y,
    int y_f32, uint32_t batch) {
    __shared__ uint32_t bits[8];
    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    __shared__ float ys[kMaxSlots][kDnRows];
    const uint32_t HID = d.hidden, IN = d.inter, TK = d.top_k;
    const uint32_t nslots = batch * TK;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if ((uint32_t)tid < nslots) {
        s_idx[tid] = idx[tid];
        s_wgt[tid] = wgt[tid];
    }
    mark_experts(s_idx, nslots, d.n_experts, bits);  // (its first barrier publishes s_idx)
    const uint32_t half = lane >> 5, c0 = lane & 31, nch = IN >> 5;
    const uint32_t m0 = blockIdx.x * kDnRows;
    constexpr int RP = kDnRows / 2;  // row pairs per wave
    const DequantConsts kc;
    uint32_t n_unique = 0;
#pragma unroll
    for (int wd = 0; wd < 8; ++wd) n_unique += __popc(bits[wd]);

    // the distinct experts, one wave each (looping when there are more)
    for (uint32_t u = wave; u < n_unique; u += kThreads / 64) {
        const Plan p = plan_for(s_idx, nslots, d.n_experts, u, bits);
        const uint8_t* proj = pool + (size_t)p.e * d.blob + d.off_down;
        uint64_t sm0 = p.m0, sm1 = p.m1;
        uint32_t slot = pop_slot(sm0, sm1);
        u32x4 raw[J][4];
        act_load<J>(H + (size_t)slot * IN, nch, c0, raw);
        u32x4 w[RP][J];
        uint32_t mt[RP][J];
#pragma unroll
        for (int r = 0; r < RP; ++r)
            load_row<J>(proj, d, IN, min(m0 + 2 * r + half, HID - 1), c0, w[r], mt[r]);
        float bi0 = 0.0f, bi1 = 0.0f;
        if (lane < RP) {
            const uint16_t* BI = reinterpret_cast<const uint16_t*>(proj + d.sub_bi);
            bi0 = bf2f(BI[min(m0 + 2 * lane, HID - 1)]);
            bi1 = bf2f(BI[min(m0 + 2 * lane + 1, HID - 1)]);
        }
        while (true) {
            Act<J> a;
            act_prep<J>(raw, a);
            const float wt = s_wgt[slot];
            float2 hs[RP];
#pragma unroll
            for (int r = 0; r < RP; ++r) hs[r] = half_sums(row_dot<J>(w[r], mt[r], a, nch, c0, kc));
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                if (lane == r) {
                    ys[slot][2 * r] = wt * (hs[r].x + bi0);
                    ys[slot][2 * r + 1] = wt * (hs[r].y + bi1);
                }
            }
            if (!(sm0 | sm1)) break;
            slot = pop_slot(sm0, sm1);
            act_load<J>(H + (size_t)slot * IN, nch, c0, raw);
        }
    }
    __syncthreads();
    // combine in slot order (moe-fused/src/kernels.metal:254-263)
    for (uint32_t i = tid; i < batch * kDnRows; i += kThreads) {
        const uint32_t t = i / kDnRows, r = i % kDnRows, m = m0 + r;
        if (m >= HID) continue;
        float acc = 0.0f;
        for (uint32_t k = 0; k < TK; ++k) acc += ys[t * TK + k][r];
        if (y_f32) reinterpret_cast<float*>(Y)[(size_t)t * HID + m] = acc;
        else reinterpret_cast<uint16_t*>(Y)[(size_t)t * HID + m] = f2h(acc);
    }
}

__global__ void fill_zero_k(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        p[i] = 0u;
}

uint32_t max_unique(const kq_moe_desc& d, uint32_t batch) {
    const uint32_t n = batch * d.top_k;
    return n < d.n_experts ? n : d.n_experts;
}

uint32_t chunks_j(uint32_t K) { return ((K >> 5) + 31) / 32; }

hipError_t launch_logits(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                         const kq_moe_desc& d, uint16_t* xh, float* lg, hipStream_t s) {
    const dim3 grid((d.n_experts + 3) / 4);
#define KQ_LG(RF, XF)                                                                           \
    moe_logits_k<RF, XF><<<grid, kThreads, 0, s>>>(R, X, batch, d.n_experts, d.hidden, xh, lg)
    if (r_f32 && x_f32) KQ_LG(true, true);
    else if (r_f32) KQ_LG(true, false);
    else if (x_f32) KQ_LG(false, true);
    else KQ_LG(false, false);
#undef KQ_LG
    return hipGetLastError();
}

template <bool FL>
hipError_t launch_gu(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx, float* wgt,
                     uint32_t* idx_pub, const float* lg, const uint16_t* xh, uint16_t* H,
                     uint32_t batch, hipStream_t s) {
    const dim3 grid((d.inter + kGuRows - 1) / kGuRows, max_unique(d, batch));
#define KQ_GU(JJ)                                                                               \
    moe_gate_up_k<JJ, FL><<<grid, kThreads, 0, s>>>(pool, d, idx, wgt, idx_pub, lg, xh, H, batch)
    switch (chunks_j(d.hidden)) {
        case 1: KQ_GU(1); break;
        case 2: KQ_GU(2); break;
        case 3: KQ_GU(3); break;
        case 4: KQ_GU(4); break;
        default: return hipErrorInvalidValue;
    }
#undef KQ_GU
    return hipGetLastError();
}

}  // namespace

size_t moe_ws_bytes(const kq_moe_desc& d, uint32_t batch) { return ws_layout(d, batch).total; }

hipError_t launch_ws_zero(void* ws, size_t bytes, hipStream_t s) {
    const size_t n = bytes / 4;
    size_t blocks = (n + 255) / 256;
    if (blocks > 1024) blocks = 1024;
    if (blocks == 0) return hipSuccess;
    fill_zero_k<<<(unsigned)blocks, 256, 0, s>>>(reinterpret_cast<uint32_t*>(ws), n);
    return hipGetLastError();
}

hipError_t launch_moe_router(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                             const kq_moe_desc& d, uint32_t* idx, float* wgt, uint16_t* xh,
                             void* ws, hipStream_t s) {
    float* lg = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + ws_layout(d, batch).lg);
    hipError_t e = launch_logits(R, r_f32, X, x_f32, batch, d, xh, lg, s);
    if (e != hipSuccess) return e;
    moe_select_k<<<1, kThreads, 0, s>>>(lg, batch, d.n_experts, d.top_k, idx, wgt);
    return hipGetLastError();
}

hipError_t launch_moe_gate_up(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                              const uint16_t* xh, uint16_t* H, uint32_t batch, hipStream_t s) {
    return launch_gu<false>(pool, d, idx, nullptr, nullptr, nullptr, xh, H, batch, s);
}

hipError_t launch_moe_down(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                           const float* wgt, const uint16_t* H, void* Y, bool y_f32,
                           uint32_t batch, hipStream_t s) {
    const dim3 grid((d.hidden + kDnRows - 1) / kDnRows);
    const int yf = y_f32 ? 1 : 0;
#define KQ_DN(JJ) moe_down_k<JJ><<<grid, kThreads, 0, s>>>(pool, d, idx, wgt, H, Y, yf, batch)
    switch (chunks_j(d.inter)) {
        case 1: KQ_DN(1); break;
        case 2: KQ_DN(2); break;
        case 3: KQ_DN(3); break;
        case 4: KQ_DN(4); break;
        default: return hipErrorInvalidValue;
    }
#undef KQ_DN
    return hipGetLastError();
}

hipError_t launch_moe_block(const uint8_t* pool, const kq_moe_desc& d, const void* R, bool r_f32,
                            const void* X, bool x_f32, uint32_t batch, uint32_t* idx, float* wgt,
                            uint16_t* xh, uint16_t* H, void* Y, bool y_f32, void* ws,
                            hipStream_t s) {
    float* lg = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) + ws_layout(d, batch).lg);
    hipError_t e = launch_logits(R, r_f32, X, x_f32, batch, d, xh, lg, s);
    if (e != hipSuccess) return e;
    const uint16_t* xin = x_f32 ? xh : reinterpret_cast<const uint16_t*>(X);
    e = launch_gu<true>(pool, d, nullptr, wgt, idx, lg, xin, H, batch, s);
    if (e != hipSuccess) return e;
    return launch_moe_down(pool, d, idx, wgt, H, Y, y_f32, batch, s);
}

}  // namespace kq
