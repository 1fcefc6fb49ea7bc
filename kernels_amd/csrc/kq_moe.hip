// kq_moe.hip -- the MoE decode block in three launches (gfx950).
//
// Reference: moe-fused/src/kernels.metal:98-265 (router_topk,
// fused_gate_up_swiglu, fused_down_combine) and the block reference
// moe-fused/src/main.mm:302-334. The block has two grid-wide dependencies
// (idx before the expert gather; all of h before down), so it is three
// kernels here too, each designed for CDNA4:
//
// 1. router_topk: the router matrix is split over many workgroups (one wave
//    per expert, all tokens of the batch per wave, so R is read once), logits
//    go to the workspace, and the last workgroup to finish (device-scope
//    counter, self-resetting) runs top-k + softmax for every token with
//    wave64 argmax butterflies. Strictly-greater-wins with an ascending scan
//    is reproduced exactly: ties go to the lowest expert index.
// 2. gate_up_swiglu: grid = (16-row tile, unique expert). Each workgroup
//    derives the ascending list of distinct selected experts from idx, takes
//    the u-th, and reads that expert's gate/up rows once for every token
//    slot that selected it. A half-wave (32 lanes) owns one projection row
//    (K = 2880 = 90 chunks -> 3 per lane), the other half the matching row of
//    the other projection, so gate and up meet in registers for SwiGLU.
// 3. down_combine: grid = (16-row tile, unique expert) again; per-slot
//    partial outputs wgt*(down.h + bias) go to the workspace and the last
//    workgroup of each row tile sums them in slot order (deterministic).
//
// Weight rows are dequantised with the AND-OR fp16 trick of kq_device.h and
// dotted against LDS-staged permuted activation pairs; the bf16 group scale
// and bias are applied once per 32-weight chunk.
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {

namespace {

constexpr int kMoeThreads = 256;
constexpr int kTileRows = 16;    // rows per workgroup (4 waves x 4 rows)
constexpr int kSlotRound = 4;    // token slots staged per LDS round

struct WsLayout {
    size_t cnt_router, cnt_tiles, lg, ys, total;
};

WsLayout ws_layout(const kq_moe_desc& d, uint32_t batch) {
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    WsLayout L;
    const size_t ntiles = (d.hidden + kTileRows - 1) / kTileRows;
    L.cnt_router = 0;
    L.cnt_tiles = 64;
    L.lg = al(L.cnt_tiles + 4 * ntiles);
    L.ys = al(L.lg + 4ull * batch * d.n_experts);
    L.total = al(L.ys + 4ull * batch * d.top_k * d.hidden);
    return L;
}

// ---------------------------------------------------------------------------
// 1. router + top-k + softmax
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

// (value, index) argmax with the reference's selection rule: a candidate is
// selectable only if strictly greater than -inf (NaN never is); among equal
// values the lower index wins.
__device__ __forceinline__ bool better(float va, uint32_t ia, float vb, uint32_t ib) {
    const bool oka = va > -INFINITY, okb = vb > -INFINITY;
    if (oka != okb) return oka;
    if (!oka) return ia < ib;
    return va > vb || (va == vb && ia < ib);
}

template <bool RF32, bool XF32>
__global__ __launch_bounds__(128) void moe_router_k(const void* __restrict__ R,
                                                    const void* __restrict__ X, uint32_t batch,
                                                    uint32_t NE, uint32_t HID, uint32_t TK,
                                                    uint32_t* __restrict__ idx,
                                                    float* __restrict__ wgt,
                                                    uint16_t* __restrict__ xh,
                                                    float* __restrict__ lg,
                                                    uint32_t* __restrict__ counter) {
    constexpr int NBMAX = 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t e = blockIdx.x * 2 + wave;

    // fp16 copy of x for the projections (router_topk writes xh the same way,
    // moe-fused/src/kernels.metal:137)
    if (XF32 && xh) {
        const uint32_t tot = batch * HID;
        for (uint32_t i = blockIdx.x * 128 + tid; i < tot; i += gridDim.x * 128)
            xh[i] = f2h(reinterpret_cast<const float*>(X)[i]);
    }

    if (e < NE) {
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

    // last-workgroup-done epilogue
    __shared__ uint32_t s_last;
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(counter, 1u) == gridDim.x - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    for (uint32_t t = wave; t < batch; t += 2) {
        const volatile float* L = lg + (size_t)t * NE;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t ei = lane + 64 * q;
            v[q] = ei < NE ? L[ei] : -INFINITY;
        }
        float chosen[8];
        uint32_t pick[8];
        for (uint32_t j = 0; j < TK; ++j) {
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
            if (!(bv > -INFINITY)) { bv = -INFINITY; bi = 0; }  // nothing selectable
            chosen[j] = bv;
            pick[j] = bi;
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if ((uint32_t)lane + 64 * q == bi) v[q] = -INFINITY;
        }
        if (lane == 0) {
            float mx = chosen[0];
            for (uint32_t j = 1; j < TK; ++j) mx = fmaxf(mx, chosen[j]);
            float sum = 0.0f, ex[8];
            for (uint32_t j = 0; j < TK; ++j) { ex[j] = expf(chosen[j] - mx); sum += ex[j]; }
            for (uint32_t j = 0; j < TK; ++j) {
                idx[t * TK + j] = pick[j];
                wgt[t * TK + j] = ex[j] / sum;
            }
        }
    }
    if (tid == 0) atomicExch(counter, 0u);
}

// ---------------------------------------------------------------------------
// shared by passes 2 and 3: the expert of work item u and its token slots
// ---------------------------------------------------------------------------
struct Plan {
    uint32_t e;         // expert id (valid if u < n_unique)
    uint32_t n_unique;  // distinct experts selected
    uint64_t m0, m1;    // slots s (s < 64: bit s of m0; else bit s-64 of m1)
};

__device__ Plan moe_plan(const uint32_t* __restrict__ idx, uint32_t nslots, uint32_t NE,
                         uint32_t u, uint32_t* bits /* LDS, 8 words */) {
    const int tid = threadIdx.x, lane = tid & 63;
    if (tid < 8) bits[tid] = 0;
    __syncthreads();
    if ((uint32_t)tid < nslots) {
        const uint32_t e = min(idx[tid], NE - 1);
        atomicOr(&bits[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
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
    const uint32_t s0 = lane, s1 = lane + 64;
    const bool q0 = s0 < nslots && min(idx[s0], NE - 1) == p.e;
    const bool q1 = s1 < nslots && min(idx[s1], NE - 1) == p.e;
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

// Stage activation vectors (fp16 [K]) of up to kSlotRound slots into LDS as
// permuted pairs [slot][word%4][chunk] and per-chunk (sum, offset const).
__device__ __forceinline__ void stage_acts(const uint16_t* base, const uint32_t* offs, int ns,
                                           uint32_t K, u32x4* xp, float2* xk) {
    const uint32_t nw = K >> 3, nch = K >> 5;
    const uint32_t total = (uint32_t)ns * nw;
    const int tid = threadIdx.x;
    for (uint32_t w0 = 0; w0 < total; w0 += kMoeThreads) {
        const uint32_t w = w0 + tid;
        const bool ok = w < total;
        const uint32_t t = ok ? w / nw : 0, wi = ok ? w - t * nw : 0;
        u32x4 v = ok ? *reinterpret_cast<const u32x4*>(base + (size_t)offs[t] + (size_t)wi * 8)
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
}

// Partial (per-lane) dot of J chunks of one row with staged activation slot t.
template <int J>
__device__ __forceinline__ float row_partial(const u32x4 (&w)[J], const uint32_t (&mt)[J],
                                             const u32x4* xp, const float2* xk, uint32_t t,
                                             uint32_t nch, uint32_t c0) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t c = c0 + 32 * j;
        if (c < nch) {
            const u32x4 p0 = xp[(t * 4 + 0) * nch + c];
            const u32x4 p1 = xp[(t * 4 + 1) * nch + c];
            const u32x4 p2 = xp[(t * 4 + 2) * nch + c];
            const u32x4 p3 = xp[(t * 4 + 3) * nch + c];
            const float2 k2 = xk[t * nch + c];
            float da = qdot8(w[j].x, p0, 0.0f);
            float db = qdot8(w[j].y, p1, 0.0f);
            da = qdot8(w[j].z, p2, da);
            db = qdot8(w[j].w, p3, db);
            const float s = bf2f(mt[j] & 0xFFFFu), b = bf2f(mt[j] >> 16);
            acc = fmaf(s, (da + db) - k2.y, fmaf(b, k2.x, acc));
        }
    }
    return acc;
}

// Load J chunks (lane c0 + 32j) of row m of a projection plus bf16 S/B.
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

// ---------------------------------------------------------------------------
// 2. gather + gate + up + SwiGLU
// ---------------------------------------------------------------------------
template <int J>
__global__ __launch_bounds__(kMoeThreads) void moe_gate_up_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx,
    const uint16_t* __restrict__ xh, uint16_t* __restrict__ H, uint32_t batch) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ uint32_t bits[8];
    const uint32_t HID = d.hidden, IN = d.inter, TK = d.top_k;
    const uint32_t nslots = batch * TK;
    const Plan p = moe_plan(idx, nslots, d.n_experts, blockIdx.y, bits);
    if (blockIdx.y >= p.n_unique) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t half = lane >> 5, c0 = lane & 31, nch = HID >> 5;
    const uint8_t* blob = pool + (size_t)p.e * d.blob;
    const uint8_t* proj = blob + (half ? d.off_up : d.off_gate);

    // issue this wave's weight loads before staging activations
    constexpr int RW = kTileRows / 4;  // rows per wave
    const uint32_t mrow0 = blockIdx.x * kTileRows + wave * RW;
    u32x4 w[RW][J];
    uint32_t mt[RW][J];
    float bias[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const uint32_t m = min(mrow0 + r, IN - 1);
        load_row<J>(proj, d, HID, m, c0, w[r], mt[r]);
        bias[r] = bf2f(reinterpret_cast<const uint16_t*>(proj + d.sub_bi)[m]);
    }

    u32x4* xp = reinterpret_cast<u32x4*>(smem);
    float2* xk = reinterpret_cast<float2*>(smem + (size_t)kSlotRound * nch * 64);
    __shared__ uint32_t s_sl[kSlotRound], s_off[kSlotRound];
    uint64_t m0 = p.m0, m1 = p.m1;
    while (m0 | m1) {
        __syncthreads();  // previous round's LDS reads are done
        int ns = 0;
        while ((m0 | m1) && ns < kSlotRound) {
            const uint32_t sl = pop_slot(m0, m1);
            if (tid == 0) { s_sl[ns] = sl; s_off[ns] = (sl / TK) * HID; }
            ++ns;
        }
        __syncthreads();
        stage_acts(xh, s_off, ns, HID, xp, xk);
        __syncthreads();
        for (int t = 0; t < ns; ++t) {
            const uint32_t slot = s_sl[t];
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                float v = group_sum<32>(row_partial<J>(w[r], mt[r], xp, xk, t, nch, c0)) + bias[r];
                const float o = __shfl_xor(v, 32, 64);
                const uint32_t m = mrow0 + r;
                if (lane == r && m < IN) {
                    const float g = fminf(v, 7.0f);  // lane < 32 holds gate
                    const float uu = fminf(fmaxf(o, -7.0f), 7.0f);
                    const float h = (g / (1.0f + expf(-1.702f * g))) * (uu + 1.0f);
                    H[(size_t)slot * IN + m] = f2h(h);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// 3. gather + down + weighted combine
// ---------------------------------------------------------------------------
template <int J>
__global__ __launch_bounds__(kMoeThreads) void moe_down_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx,
    const float* __restrict__ wgt, const uint16_t* __restrict__ H, void* __restrict__ Y,
    int y_f32, uint32_t batch, float* __restrict__ ys, uint32_t* __restrict__ tile_cnt) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ uint32_t bits[8];
    __shared__ uint32_t s_last;
    const uint32_t HID = d.hidden, IN = d.inter, TK = d.top_k;
    const uint32_t nslots = batch * TK;
    const Plan p = moe_plan(idx, nslots, d.n_experts, blockIdx.y, bits);
    if (blockIdx.y >= p.n_unique) return;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t half = lane >> 5, c0 = lane & 31, nch = IN >> 5;
    const uint8_t* proj = pool + (size_t)p.e * d.blob + d.off_down;

    // wave rows: pairs (2q, 2q+1), the half-wave picks one of the pair
    constexpr int RP = kTileRows / 8;  // row pairs per wave
    const uint32_t mrow0 = blockIdx.x * kTileRows + wave * (2 * RP);
    u32x4 w[RP][J];
    uint32_t mt[RP][J];
    float bias[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        const uint32_t m = min(mrow0 + 2 * r + half, HID - 1);
        load_row<J>(proj, d, IN, m, c0, w[r], mt[r]);
        bias[r] = bf2f(reinterpret_cast<const uint16_t*>(proj + d.sub_bi)[m]);
    }

    u32x4* xp = reinterpret_cast<u32x4*>(smem);
    float2* xk = reinterpret_cast<float2*>(smem + (size_t)kSlotRound * nch * 64);
    __shared__ uint32_t s_sl[kSlotRound], s_off[kSlotRound];
    uint64_t m0 = p.m0, m1 = p.m1;
    while (m0 | m1) {
        __syncthreads();
        int ns = 0;
        while ((m0 | m1) && ns < kSlotRound) {
            const uint32_t sl = pop_slot(m0, m1);
            if (tid == 0) { s_sl[ns] = sl; s_off[ns] = sl * IN; }
            ++ns;
        }
        __syncthreads();
        stage_acts(H, s_off, ns, IN, xp, xk);
        __syncthreads();
        for (int t = 0; t < ns; ++t) {
            const uint32_t slot = s_sl[t];
            const float wt = wgt[slot];
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                const float v = group_sum<32>(row_partial<J>(w[r], mt[r], xp, xk, t, nch, c0));
                const uint32_t m = mrow0 + 2 * r + half;
                if (c0 == 0 && m < HID) ys[(size_t)slot * HID + m] = wt * (v + bias[r]);
            }
        }
    }

    // the last of the n_unique workgroups of this row tile combines in slot order
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&tile_cnt[blockIdx.x], 1u) == p.n_unique - 1);
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const uint32_t mt0 = blockIdx.x * kTileRows;
    for (uint32_t i = tid; i < batch * kTileRows; i += kMoeThreads) {
        const uint32_t t = i / kTileRows, m = mt0 + i % kTileRows;
        if (m >= HID) continue;
        const volatile float* yv = ys + (size_t)t * TK * HID + m;
        float acc = 0.0f;
        for (uint32_t k = 0; k < TK; ++k) acc += yv[(size_t)k * HID];
        if (y_f32) reinterpret_cast<float*>(Y)[(size_t)t * HID + m] = acc;
        else reinterpret_cast<uint16_t*>(Y)[(size_t)t * HID + m] = f2h(acc);
    }
    if (tid == 0) atomicExch(&tile_cnt[blockIdx.x], 0u);
}

__global__ void fill_zero_k(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        p[i] = 0u;
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
    const WsLayout L = ws_layout(d, batch);
    uint8_t* w = reinterpret_cast<uint8_t*>(ws);
    float* lg = reinterpret_cast<float*>(w + L.lg);
    uint32_t* cnt = reinterpret_cast<uint32_t*>(w + L.cnt_router);
    const dim3 grid((d.n_experts + 1) / 2);
#define KQ_ROUTER(RF, XF)                                                                       \
    moe_router_k<RF, XF><<<grid, 128, 0, s>>>(R, X, batch, d.n_experts, d.hidden, d.top_k, idx, \
                                              wgt, xh, lg, cnt)
    if (r_f32 && x_f32) KQ_ROUTER(true, true);
    else if (r_f32) KQ_ROUTER(true, false);
    else if (x_f32) KQ_ROUTER(false, true);
    else KQ_ROUTER(false, false);
#undef KQ_ROUTER
    return hipGetLastError();
}

static uint32_t max_unique(const kq_moe_desc& d, uint32_t batch) {
    const uint32_t n = batch * d.top_k;
    return n < d.n_experts ? n : d.n_experts;
}

hipError_t launch_moe_gate_up(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                              const uint16_t* xh, uint16_t* H, uint32_t batch, hipStream_t s) {
    const uint32_t J = ((d.hidden >> 5) + 31) / 32;
    const dim3 grid((d.inter + kTileRows - 1) / kTileRows, max_unique(d, batch));
    const size_t lds = (size_t)kSlotRound * (d.hidden >> 5) * 72;
    switch (J) {
        case 1: moe_gate_up_k<1><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, xh, H, batch); break;
        case 2: moe_gate_up_k<2><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, xh, H, batch); break;
        case 3: moe_gate_up_k<3><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, xh, H, batch); break;
        case 4: moe_gate_up_k<4><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, xh, H, batch); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_moe_down(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                           const float* wgt, const uint16_t* H, void* Y, bool y_f32,
                           uint32_t batch, void* ws, hipStream_t s) {
    const WsLayout L = ws_layout(d, batch);
    uint8_t* w = reinterpret_cast<uint8_t*>(ws);
    float* ys = reinterpret_cast<float*>(w + L.ys);
    uint32_t* tc = reinterpret_cast<uint32_t*>(w + L.cnt_tiles);
    const uint32_t J = ((d.inter >> 5) + 31) / 32;
    const dim3 grid((d.hidden + kTileRows - 1) / kTileRows, max_unique(d, batch));
    const size_t lds = (size_t)kSlotRound * (d.inter >> 5) * 72;
    const int yf = y_f32 ? 1 : 0;
    switch (J) {
        case 1: moe_down_k<1><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, wgt, H, Y, yf, batch, ys, tc); break;
        case 2: moe_down_k<2><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, wgt, H, Y, yf, batch, ys, tc); break;
        case 3: moe_down_k<3><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, wgt, H, Y, yf, batch, ys, tc); break;
        case 4: moe_down_k<4><<<grid, kMoeThreads, lds, s>>>(pool, d, idx, wgt, H, Y, yf, batch, ys, tc); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace kq
