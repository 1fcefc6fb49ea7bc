// kq_moe.hip -- the MoE decode block (gfx950).
//
// Reference: moe-fused/src/kernels.metal:98-265 (router_topk,
// fused_gate_up_swiglu, fused_down_combine) and the block reference
// moe-fused/src/main.mm:302-334. Three launches, as in the reference:
//
// 1. moe_router_k: router logits (one wave per expert, fp32 accumulation,
//    every load issued before the first multiply), then the workgroup that
//    completes last (a device-scope counter) runs top-k + softmax for every
//    token and publishes idx, wgt and a plan: the ascending list of distinct
//    selected experts and, per expert, the token slots that chose it. The
//    logits travel through device-coherent stores and loads (relaxed
//    agent-scope atomics: they bypass the non-coherent per-XCD L2), so no
//    L2 write-back fence is needed -- measured ~2 us cheaper per block than a
//    release fence, and cheaper than a separate selection launch.
//    At 1-2 tokens the block's router stops after the logits instead: every
//    wave of the streaming gate/up launch runs the top-k and builds the plan
//    itself (no barrier before its weight loads), and workgroup 0 publishes
//    idx, wgt and the plan for down.
// 2. gate/up + SwiGLU, and 3. down + weighted combine, in these forms:
//    - streaming (moe_gu_stream_k up to 2 tokens, moe_dn_stream_k while the
//      slots' h vectors fit in LDS, up to 5 tokens at gpt-oss shapes): one
//      workgroup per CU, each wave streams (expert, row pair) items through
//      a 2-deep ring of register slots, compute overlapped with the next
//      item's loads; the activations are prepared once per workgroup in LDS
//      (at one token, held in registers); down keeps per-slot
//      wgt * (down . h + bias) in LDS and sums the slots in k order;
//    - expert-partitioned (the block's gate/up from 3 tokens, moe_gu_part_k;
//      its down from 6 tokens, moe_dn_part_k): one round of one workgroup
//      per CU; each plan entry gets workgroups in proportion to its cost
//      (rows x (4 + 3 x slots)), and a workgroup streams a row chunk of one
//      expert with only that expert's activations in LDS; down writes
//      per-slot products to the workspace and a small moe_combine_k launch
//      sums them in slot order (4 launches in all);
//    - per tile (moe_gate_up_k, moe_down_k): the standalone entry points
//      past the streaming limits (they take no workspace): a grid of
//      (16-row tile, expert) or 8-output-row workgroups that issue all of
//      their loads in one round trip.
//    Every form reads each selected expert's rows once per call for all
//    token slots that chose it; a half-wave owns one row of a pair (gate /
//    up, or two down rows; K = 2880 = 90 chunks -> 3 per lane), so SwiGLU
//    and the combine see the two half sums. Sums are deterministic (fixed
//    order, no atomics).
//
// Activations are used as permuted fp16 pairs with per-chunk sums (the
// AND-OR dequant of kq_device.h); bf16 group scale and bias apply once per
// 32-weight chunk.
#include <mutex>
#include <type_traits>

#include "kq_device.h"
#include "kq_internal.h"
#include "kq_moe_device.h"

namespace kq {

// Workspace of kq_moe_block_noalloc: one array per GPU in the code object's
// own device memory, held until the process ends. Host code never passes
// `scratch` itself to a kernel (on the host the name is only a stand-in for
// the symbol); it uses the per-device address hipGetSymbolAddress returns.
static __device__ __align__(256) uint8_t scratch[KQ_MOE_NOALLOC_WS_BYTES];

namespace {

constexpr int kMaxSlots = 128;  // batch (16) x top_k (8)
constexpr int kMaxTopK = 8;
constexpr int kGuThreads = 256;  // gate/up: 4 waves
constexpr int kGuRW = 4;         // gate/up rows per wave
constexpr int kGuRows = 16;      // gate/up rows per workgroup
constexpr int kDnThreads = 256;  // down: 4 waves
constexpr int kDnRows = 8;       // down rows per workgroup

// Plan of one call: distinct selected experts (ascending) and their slots.
struct Plan {
    uint32_t n;
    uint32_t pad[3];
    uint32_t expert[kMaxSlots];
    uint64_t mask[kMaxSlots][2];  // slot s: bit s of mask[.][0] (s < 64) or bit s-64 of [1]
};

struct WsLayout {
    size_t lg, cnt, plan, sync, tag, ys, xsh, total;
};

// Workspace: [completion counter, error word][plan][grid-barrier counters]
// [tagged logits of the one-launch block, kTagCopies x 8 B x 256][logits f32 batch x
// n_experts][per-slot down products f32 batch x top_k x hidden][the atomic
// block's sum(h) per slot and 32-chunk, f32 batch x top_k x ceil(inter / 32)]. Everything
// before the logits sits at fixed offsets, the same for every batch and
// descriptor: a workspace sized for a large batch and reused at a smaller
// one (or the reverse) never has its counter, plan or barrier state
// overwritten by another call's logits or products. Every call writes the
// logits and products it reads.
constexpr size_t kWsCnt = 0, kWsPlan = 256;
constexpr uint32_t kSyncGroups = 32;  // barrier counters: workgroups b % 32 (8 per counter at 256)
constexpr size_t kSyncStride = 256;  // bytes between counters (separate lines)
constexpr size_t kWsSync = (kWsPlan + sizeof(Plan) + 255) & ~(size_t)255;
constexpr size_t kWsTag = kWsSync + kSyncGroups * kSyncStride;
constexpr uint32_t kTagCopies = 8;  // one per XCD (workgroups b % 8)
WsLayout ws_layout(const kq_moe_desc& d, uint32_t batch) {
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    WsLayout L;
    L.cnt = kWsCnt;
    L.plan = kWsPlan;
    L.sync = kWsSync;
    L.tag = kWsTag;
    L.lg = L.tag + kTagCopies * 8 * 256;
    L.ys = L.lg + al(4ull * batch * d.n_experts);
    L.xsh = L.ys + al(4ull * batch * d.top_k * d.hidden);
    L.total = L.xsh + al(4ull * batch * d.top_k * ((d.inter + 31) / 32));
    return L;
}

// Valid slot bits of a plan mask word h for nslots slots: a plan read from
// the workspace is masked with these, so no slot index it yields reaches
// past the call's nslots slots (wgt, H, ys and the LDS blocks).
__device__ __forceinline__ uint64_t slot_bits(uint32_t nslots, int h) {
    const uint32_t n = h ? (nslots > 64 ? nslots - 64 : 0) : (nslots < 64 ? nslots : 64);
    return n >= 64 ? ~0ull : ((1ull << n) - 1ull);
}

// Eight consecutive elements as loaded (fp16: one u32x4; fp32: two f32x4).
template <bool F32>
struct Raw8;
template <>
struct Raw8<false> {
    u32x4 v;
};
template <>
struct Raw8<true> {
    f32x4 a, b;
};

template <bool F32>
__device__ __forceinline__ Raw8<F32> load8(const void* p, size_t i) {
    Raw8<F32> r;
    if constexpr (F32) {
        const f32x4* q = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + i);
        r.a = q[0];
        r.b = q[1];
    } else {
        r.v = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(p) + i);
    }
    return r;
}

template <bool F32>
__device__ __forceinline__ void unpack8(const Raw8<F32>& r, float v[8]) {
    if constexpr (F32) {
        v[0] = r.a.x; v[1] = r.a.y; v[2] = r.a.z; v[3] = r.a.w;
        v[4] = r.b.x; v[5] = r.b.y; v[6] = r.b.z; v[7] = r.b.w;
    } else {
        v[0] = h2f(r.v.x & 0xFFFF); v[1] = h2f(r.v.x >> 16);
        v[2] = h2f(r.v.y & 0xFFFF); v[3] = h2f(r.v.y >> 16);
        v[4] = h2f(r.v.z & 0xFFFF); v[5] = h2f(r.v.z >> 16);
        v[6] = h2f(r.v.w & 0xFFFF); v[7] = h2f(r.v.w >> 16);
    }
}

// top-k + softmax of one token, one wave (moe-fused/src/kernels.metal:149-162):
// the selection of topk_select over the token's logits (4 per lane), then
// the softmax of the selected logits. COHERENT: the logits come from other
// workgroups of the same launch (device-coherent loads); otherwise from an
// earlier launch (plain loads).
// topk_vals: the same from the logits already in registers (lane l holds
// experts l + 64q in x[q]). topk_lanes: the same results in registers, slot
// j's expert and weight in lane j (lanes from TK on: expert 0, weight 0).
__device__ __forceinline__ void topk_lanes(const float (&x)[4], uint32_t NE, uint32_t TK,
                                           uint32_t& pj, float& wj);
__device__ __forceinline__ void topk_vals(const float (&x)[4], uint32_t NE, uint32_t TK,
                                          uint32_t* idx_out, float* wgt_out);
template <bool COHERENT>
__device__ __forceinline__ void topk_wave(const float* L, uint32_t NE, uint32_t TK,
                          uint32_t* idx_out, float* wgt_out) {
    const uint32_t lane = threadIdx.x & 63;
    float x[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t ei = lane + 64 * q;
        if constexpr (COHERENT)
            x[q] = __hip_atomic_load(L + min(ei, NE - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
            x[q] = L[min(ei, NE - 1)];
    }
    topk_vals(x, NE, TK, idx_out, wgt_out);
}
__device__ __forceinline__ void topk_lanes(const float (&x)[4], uint32_t NE, uint32_t TK,
                                           uint32_t& pj, float& wj) {
    const uint32_t lane = threadIdx.x & 63;
    float v[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) v[q] = cand(x[q], lane + 64 * q < NE);
    float chosen[kMaxTopK];
    uint32_t pick[kMaxTopK];
    topk_select(v, TK, pick, chosen);
    // softmax over the selected logits, slot j in lane j: one exp per lane and
    // a three-step sum instead of a serial chain in one lane. The passes pick
    // in descending order, so the largest selected logit is chosen[0].
    const float mx = chosen[0];
    float cj = -INFINITY;
    pj = 0;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if ((uint32_t)j < TK && lane == (uint32_t)j) {
            cj = chosen[j];
            pj = pick[j];
        }
    }
    const float ex = lane < TK ? __expf(cj - mx) : 0.0f;
    // lanes 0-7 each get ((e0 + e1) + (e2 + e3)) + ((e4 + e5) + (e6 + e7)):
    // partners xor 1 and xor 2 by quad permutes, then the other quad of the
    // 8-lane half-row by its mirror (lane 7 - i, whose quad holds that sum)
    float sum = ex;
    sum = dpp_fadd<0xB1>(sum);   // quad_perm [1,0,3,2]
    sum = dpp_fadd<0x4E>(sum);   // quad_perm [2,3,0,1]
    sum = dpp_fadd<0x141>(sum);  // row_half_mirror
    wj = lane < TK ? __fdividef(ex, sum) : 0.0f;
}
__device__ __forceinline__ void topk_vals(const float (&x)[4], uint32_t NE, uint32_t TK,
                                          uint32_t* idx_out, float* wgt_out) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t pj;
    float wj;
    topk_lanes(x, NE, TK, pj, wj);
    if (lane < TK) {
        idx_out[lane] = pj;
        wgt_out[lane] = wj;
    }
}

// ---------------------------------------------------------------------------
// 1. router logits + (last workgroup) top-k and plan
// ---------------------------------------------------------------------------
// Plan of the slots s_idx[0 .. nslots) into ps (all threads of the workgroup).
__device__ void build_plan(const uint32_t* s_idx, uint32_t nslots, uint32_t NE, Plan& ps,
                           uint32_t* bits) {
    // O(1) per thread: mark the selected experts, rank each slot's expert by
    // the marks below it, OR the slot into its entry's mask
    const uint32_t tid = threadIdx.x;
    if (tid < 8) bits[tid] = 0;
    for (uint32_t i = tid; i < 2 * kMaxSlots; i += blockDim.x) ps.mask[i >> 1][i & 1] = 0;
    __syncthreads();
    uint32_t e = 0;
    if (tid < nslots) {
        e = min(s_idx[tid], NE - 1);
        atomicOr(&bits[e >> 5], 1u << (e & 31));
    }
    __syncthreads();
    if (tid < nslots) {
        const uint32_t w = e >> 5, b = e & 31;
        uint32_t rank = __popc(bits[w] & ((1u << b) - 1u));
        for (uint32_t i = 0; i < w; ++i) rank += __popc(bits[i]);
        ps.expert[rank] = e;  // every slot of the expert writes the same value
        atomicOr(reinterpret_cast<unsigned long long*>(&ps.mask[rank][tid >> 6]),
                 1ull << (tid & 63));
    }
    if (tid == 0) {
        uint32_t n = 0;
        for (int i = 0; i < 8; ++i) n += __popc(bits[i]);
        ps.n = n;
    }
    __syncthreads();
}

// Wave w of workgroup (x, y): expert 4x + w, tokens 2y, 2y + 1. Lane l takes
// elements 8(l + 64i), i < IT (IT * 512 >= hidden); every router and x load
// is issued before the first multiply (addresses clamped, results past the
// row masked), so a wave pays one memory round trip.
template <bool RF32, bool XF32, int IT, bool TAIL, int NW>
__global__ __launch_bounds__(64 * NW) void moe_router_k(
    const void* __restrict__ R, const void* __restrict__ X, uint32_t batch, uint32_t NE,
    uint32_t HID, uint32_t TK, uint16_t* __restrict__ xh, float* lg, uint32_t* cnt,
    uint32_t* __restrict__ idx_out, float* __restrict__ wgt_out, Plan* __restrict__ plan_out,
    float* __restrict__ xsz = nullptr, uint32_t nxs = 0) {
    constexpr int NBT = 2;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t e = blockIdx.x * (NW) + wave, ec = min(e, NE - 1);
    const uint32_t t0 = blockIdx.y * NBT;
    Raw8<RF32> r[IT];
    Raw8<XF32> x[NBT][IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
        const uint32_t k = min((lane + 64 * i) * 8, HID - 8);
        r[i] = load8<RF32>(R, (size_t)ec * HID + k);
#pragma unroll
        for (int t = 0; t < NBT; ++t)
            x[t][i] = load8<XF32>(X, (size_t)min(t0 + t, batch - 1) * HID + k);
    }
    if (xsz) {  // the atomic block's sum(h) accumulators, zeroed as the reference's pass 1 does
        const uint32_t nthr = gridDim.x * gridDim.y * (64 * NW);
        for (uint32_t i = (blockIdx.y * gridDim.x + blockIdx.x) * (64 * NW) + tid; i < nxs; i += nthr)
            xsz[i] = 0.0f;
    }
    if (XF32 && xh) {  // fp16 copy of x for the projections, spread over the grid
        const uint32_t tot = batch * HID, nthr = gridDim.x * gridDim.y * (64 * NW);
        for (uint32_t i = (blockIdx.y * gridDim.x + blockIdx.x) * (64 * NW) + tid; i < tot;
             i += nthr)
            xh[i] = f2h(reinterpret_cast<const float*>(X)[i]);
    }
    float acc[NBT] = {};
#pragma unroll
    for (int i = 0; i < IT; ++i) {
        if ((lane + 64 * i) * 8 < HID) {
            float rv[8];
            unpack8<RF32>(r[i], rv);
#pragma unroll
            for (int t = 0; t < NBT; ++t) {
                float xv[8];
                unpack8<XF32>(x[t][i], xv);
                float a = acc[t];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = fmaf(rv[q], xv[q], a);
                acc[t] = a;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < NBT; ++t) {
        const float v = wave_sum(acc[t]);
        if (lane == 0 && e < NE && t0 + t < batch)
            __hip_atomic_store(lg + (size_t)(t0 + t) * NE + e, v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    // without the tail, the next launch runs the top-k from the logits
    if constexpr (!TAIL) return;
    // this workgroup's logits have reached the device-coherent level before
    // it is counted; the last one counted sees every logit
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __shared__ uint32_t s_last;
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                 gridDim.x * gridDim.y - 1;
    __syncthreads();
    if (!s_last) return;

    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    __shared__ uint32_t bits[8];
    __shared__ Plan ps;
    for (uint32_t t = wave; t < batch; t += NW)
        topk_wave<true>(lg + (size_t)t * NE, NE, TK, s_idx + t * TK, s_wgt + t * TK);
    __syncthreads();
    const uint32_t nslots = batch * TK;
    if (tid < nslots) {
        idx_out[tid] = s_idx[tid];
        wgt_out[tid] = s_wgt[tid];
    }
    build_plan(s_idx, nslots, NE, ps, bits);
    if (plan_out) {
        const uint32_t n = ps.n;
        if (tid == 0) plan_out->n = n;
        for (uint32_t u = tid; u < n; u += (64 * NW)) {
            plan_out->expert[u] = ps.expert[u];
            plan_out->mask[u][0] = ps.mask[u][0];
            plan_out->mask[u][1] = ps.mask[u][1];
        }
    }
    if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t pop_slot(uint64_t& m0, uint64_t& m1) {
    if (m0) { const uint32_t s = __builtin_ctzll(m0); m0 &= m0 - 1; return s; }
    const uint32_t s = 64 + __builtin_ctzll(m1);
    m1 &= m1 - 1;
    return s;
}

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
// Scale and bias stay as loaded (zero-extended halves) until the compute
// uses them: combining them right after the load would make the wave wait
// for every load in flight (vmcnt retires in order).
template <int J>
struct Row {
    u32x4 w[J];
    uint16_t s[J], b[J];  // bf16 bits, widened at use
};

template <int J>
__device__ __forceinline__ void load_row(const uint8_t* proj, const kq_moe_desc& d, uint32_t K,
                                         uint32_t m, uint32_t c0, Row<J>& row) {
    const uint32_t nch = K >> 5, gpr = K >> 6;
    const u32x4* W = reinterpret_cast<const u32x4*>(proj + d.sub_w) + (size_t)m * nch;
    const uint16_t* S = reinterpret_cast<const uint16_t*>(proj + d.sub_s) + (size_t)m * gpr;
    const uint16_t* B = reinterpret_cast<const uint16_t*>(proj + d.sub_b) + (size_t)m * gpr;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t c = min(c0 + 32 * j, nch - 1);
        row.w[j] = ldg_nt(W + c);
        row.s[j] = S[c >> 1];
        row.b[j] = B[c >> 1];
    }
}

// Per-lane partial dot of one row's J chunks with a register activation.
// The rows stay in registers while a wave walks its token slots, so the
// dequantisation is loop-invariant; the empty asm makes each chunk opaque at
// its use, which keeps the compiler from hoisting the dequant of every row to
// right after its load (a wait on every load, and ~200 registers of results).
template <int J>
__device__ __forceinline__ float row_dot(const Row<J>& row, const Act<J>& a, uint32_t nch,
                                         uint32_t c0, const DequantConsts& kc) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        u32x4 w = row.w[j];
        uint32_t sr = row.s[j], br = row.b[j];
        asm volatile("" : "+v"(w), "+v"(sr), "+v"(br));
        if (c0 + 32 * j < nch) {
            float da = qdot8(w.x, a.p[j][0], 0.0f, kc);
            float db = qdot8(w.y, a.p[j][1], 0.0f, kc);
            da = qdot8(w.z, a.p[j][2], da, kc);
            db = qdot8(w.w, a.p[j][3], db, kc);
            const float s = bf2f((uint16_t)sr), b = bf2f((uint16_t)br);
            acc = fmaf(s, (da + db) - a.xc[j], fmaf(b, a.xs[j], acc));
        }
    }
    return acc;
}

// ---------------------------------------------------------------------------
// plan and activations in LDS (gate/up and down)
// ---------------------------------------------------------------------------
// Loads the plan (from the router) or builds it from idx; wgt to LDS if given.
template <bool FROM_PLAN>
__device__ void get_plan(const Plan* plan_g, const uint32_t* idx, const float* wgt,
                         uint32_t nslots, uint32_t NE, Plan& ps, uint32_t* s_idx, float* s_wgt,
                         uint32_t* bits) {
    const uint32_t tid = threadIdx.x;
    if (tid < nslots) {
        s_idx[tid] = idx[tid];
        if (wgt) s_wgt[tid] = wgt[tid];
    }
    if constexpr (FROM_PLAN) {
        const uint32_t n = min(plan_g->n, nslots);
        if (tid == 0) ps.n = n;
        for (uint32_t u = tid; u < n; u += blockDim.x) {
            ps.expert[u] = plan_g->expert[u];
            ps.mask[u][0] = plan_g->mask[u][0] & slot_bits(nslots, 0);
            ps.mask[u][1] = plan_g->mask[u][1] & slot_bits(nslots, 1);
        }
        __syncthreads();
    } else {
        __syncthreads();
        build_plan(s_idx, nslots, NE, ps, bits);
    }
}

// The router's tail run by every wave of the next launch: top-k + softmax of
// every token from the logits lg, then the plan. Every wave computes the same
// values and writes the same LDS words, so each wave can use its own results
// without a workgroup barrier and issue its weight loads at once (wave 0
// alone with the other waves at a barrier measured 0.2 us slower per block,
// though the two waves of a SIMD then do not compete for issue). The plan
// lists the distinct experts in the order of their first slot (the down
// launch reads the same plan, so any fixed order gives the same result):
// at one token the top-k experts are distinct and slot s is plan entry s.
// At most kPlanSlots slots (the launcher's limit), lane s takes slot s.
// COHERENT: the logits were written by other workgroups of the same launch.
constexpr uint32_t kPlanSlots = 2 * kMaxTopK;
template <bool COHERENT = false>
__device__ __forceinline__ void plan_from_logits(const float* lg, uint32_t batch, uint32_t NE, uint32_t TK,
                                 Plan& ps, uint32_t* s_idx, float* s_wgt) {
    const uint32_t lane = threadIdx.x & 63;
    for (uint32_t t = 0; t < batch; ++t)
        topk_wave<COHERENT>(lg + (size_t)t * NE, NE, TK, s_idx + t * TK, s_wgt + t * TK);
    __builtin_amdgcn_wave_barrier();
    const uint32_t nslots = batch * TK;
    const uint32_t e = lane < nslots ? min(s_idx[lane], NE - 1) : 0xFFFFFFFFu;
    bool first = lane < nslots;
    uint64_t m = first ? 1ull << lane : 0ull;
    if (batch > 1) {  // later tokens may repeat an expert: one plan entry per expert
        m = 0;
        for (uint32_t s2 = 0; s2 < nslots; ++s2) {
            const uint32_t e2 = __builtin_amdgcn_readlane(e, s2);
            if (e2 == e) {
                m |= 1ull << s2;
                if (s2 < lane) first = false;
            }
        }
    }
    const uint64_t firsts = __ballot(first);
    if (first) {
        const uint32_t rank = __popcll(firsts & ((1ull << lane) - 1ull));
        ps.expert[rank] = e;
        ps.mask[rank][0] = m;
        ps.mask[rank][1] = 0;
    }
    if (lane == 0) ps.n = __popcll(firsts);
    __builtin_amdgcn_wave_barrier();
}

// Workgroup 0 of the gate/up launch publishes idx, wgt and the plan for the
// down launch (after its own weight loads are issued).
__device__ void publish_plan(const Plan& ps, const uint32_t* s_idx, const float* s_wgt,
                             uint32_t nslots, uint32_t* idx_out, float* wgt_out,
                             Plan* plan_out) {
    const uint32_t tid = threadIdx.x;
    if (tid < nslots) {
        idx_out[tid] = s_idx[tid];
        wgt_out[tid] = s_wgt[tid];
    }
    const uint32_t n = ps.n;
    if (tid == 0) plan_out->n = n;
    for (uint32_t u = tid; u < n; u += blockDim.x) {
        plan_out->expert[u] = ps.expert[u];
        plan_out->mask[u][0] = ps.mask[u][0];
        plan_out->mask[u][1] = ps.mask[u][1];
    }
}

// ---------------------------------------------------------------------------
// 2. gather + gate + up + SwiGLU
// ---------------------------------------------------------------------------
// Grid (16-row tile, u): workgroup (x, u) takes the u-th distinct selected
// expert of the plan, wave w rows 16x + 4w .. +3, and issues every load it
// needs at once (x of its first slot, 4 gate + 4 up rows, biases): one memory
// round trip, with the whole matrix in flight over the grid. Each row group is
// then applied to every token slot that chose the expert.
template <int J, bool FROM_PLAN>
__global__ __launch_bounds__(kGuThreads) void moe_gate_up_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx,
    const Plan* __restrict__ plan_g, const uint16_t* __restrict__ xh, uint16_t* __restrict__ H,
    uint32_t batch) {
    const uint32_t HID = d.hidden, IN = d.inter, TK = d.top_k, nch = HID >> 5;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t half = lane >> 5, c0 = lane & 31, u = blockIdx.y;
    uint32_t e, n;
    uint64_t sm0, sm1;
    if constexpr (FROM_PLAN) {
        n = min(plan_g->n, batch * TK);
        e = plan_g->expert[min(u, (uint32_t)kMaxSlots - 1)];
        sm0 = plan_g->mask[min(u, (uint32_t)kMaxSlots - 1)][0] & slot_bits(batch * TK, 0);
        sm1 = plan_g->mask[min(u, (uint32_t)kMaxSlots - 1)][1] & slot_bits(batch * TK, 1);
    } else {
        __shared__ Plan ps;
        __shared__ uint32_t s_idx[kMaxSlots];
        __shared__ float s_wgt[kMaxSlots];
        __shared__ uint32_t bits[8];
        get_plan<false>(nullptr, idx, nullptr, batch * TK, d.n_experts, ps, s_idx, s_wgt, bits);
        n = ps.n;
        e = ps.expert[u];
        sm0 = ps.mask[u][0];
        sm1 = ps.mask[u][1];
    }
    if (u >= n) return;
    e = min(e, d.n_experts - 1);

    const uint8_t* blob = pool + (size_t)e * d.blob;
    const uint8_t* proj = blob + (half ? d.off_up : d.off_gate);
    const uint32_t m0 = blockIdx.x * kGuRows + wave * kGuRW;
    const DequantConsts kc;

    uint32_t slot = pop_slot(sm0, sm1);
    u32x4 raw[J][4];
    act_load<J>(xh + (size_t)(slot / TK) * HID, nch, c0, raw);
    Row<J> rows[kGuRW];
#pragma unroll
    for (int r = 0; r < kGuRW; ++r) load_row<J>(proj, d, HID, min(m0 + r, IN - 1), c0, rows[r]);
    const uint32_t brow = min(m0 + (lane & (kGuRW - 1)), IN - 1);
    const uint32_t bg_raw = reinterpret_cast<const uint16_t*>(blob + d.off_gate + d.sub_bi)[brow];
    const uint32_t bu_raw = reinterpret_cast<const uint16_t*>(blob + d.off_up + d.sub_bi)[brow];

    while (true) {
        Act<J> a;
        act_prep<J>(raw, a);
        float g[kGuRW], up[kGuRW];
#pragma unroll
        for (int r = 0; r < kGuRW; ++r) {
            const float2 hs = half_sums(row_dot<J>(rows[r], a, nch, c0, kc));
            g[r] = hs.x;
            up[r] = hs.y;
        }
#pragma unroll
        for (int r = 0; r < kGuRW; ++r) {
            if (lane == (uint32_t)r && m0 + r < IN) {
                const float h = swiglu(g[r] + bf2f((uint16_t)bg_raw), up[r] + bf2f((uint16_t)bu_raw));
                H[(size_t)slot * IN + m0 + r] = f2h(h);
            }
        }
        if (!(sm0 | sm1)) break;
        slot = pop_slot(sm0, sm1);
        act_load<J>(xh + (size_t)(slot / TK) * HID, nch, c0, raw);
    }
}

// ---------------------------------------------------------------------------
// 3. gather + down + weighted combine
// ---------------------------------------------------------------------------
template <int J, bool FROM_PLAN>
__global__ __launch_bounds__(kDnThreads) void moe_down_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx,
    const float* __restrict__ wgt, const Plan* __restrict__ plan_g,
    const uint16_t* __restrict__ H, void* __restrict__ Y, int y_f32, uint32_t batch) {
    __shared__ Plan ps;
    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    __shared__ uint32_t bits[8];
    __shared__ float ys[kMaxSlots][kDnRows];
    constexpr int RP = kDnRows / 2;  // row pairs: lanes 0-31 row 2r, lanes 32-63 row 2r + 1
    const uint32_t HID = d.hidden, IN = d.inter, TK = d.top_k, nslots = batch * TK;
    const uint32_t nch = IN >> 5;
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t half = lane >> 5, c0 = lane & 31;
    const uint32_t m0 = blockIdx.x * kDnRows;

    get_plan<FROM_PLAN>(plan_g, idx, wgt, nslots, d.n_experts, ps, s_idx, s_wgt, bits);
    const DequantConsts kc;
    // a wave takes experts wave, wave + 4, ...: the first slot's h, then all
    // the expert's rows of this workgroup, in one batch of loads
    for (uint32_t u = wave; u < ps.n; u += kDnThreads / 64) {
        const uint8_t* proj = pool + (size_t)ps.expert[u] * d.blob + d.off_down;
        uint64_t sm0 = ps.mask[u][0], sm1 = ps.mask[u][1];
        uint32_t s = pop_slot(sm0, sm1);
        u32x4 raw[J][4];
        act_load<J>(H + (size_t)s * IN, nch, c0, raw);
        Row<J> rows[RP];
#pragma unroll
        for (int r = 0; r < RP; ++r)
            load_row<J>(proj, d, IN, min(m0 + 2 * r + half, HID - 1), c0, rows[r]);
        const uint16_t* BI = reinterpret_cast<const uint16_t*>(proj + d.sub_bi);
        const uint32_t br = m0 + 2 * (lane & (RP - 1));
        const uint32_t b0 = BI[min(br, HID - 1)], b1 = BI[min(br + 1, HID - 1)];
        while (true) {
            Act<J> a;
            act_prep<J>(raw, a);
            const float wt = s_wgt[s];
            float2 hs[RP];
#pragma unroll
            for (int r = 0; r < RP; ++r) hs[r] = half_sums(row_dot<J>(rows[r], a, nch, c0, kc));
#pragma unroll
            for (int r = 0; r < RP; ++r) {
                if (lane == (uint32_t)r) {
                    ys[s][2 * r] = wt * (hs[r].x + bf2f((uint16_t)b0));
                    ys[s][2 * r + 1] = wt * (hs[r].y + bf2f((uint16_t)b1));
                }
            }
            if (!(sm0 | sm1)) break;
            s = pop_slot(sm0, sm1);
            act_load<J>(H + (size_t)s * IN, nch, c0, raw);
        }
    }
    __syncthreads();
    // combine in slot order (moe-fused/src/kernels.metal:254-263)
    for (uint32_t i = tid; i < batch * kDnRows; i += kDnThreads) {
        const uint32_t t = i / kDnRows, r = i % kDnRows, m = m0 + r;
        if (m >= HID) continue;
        float acc = 0.0f;
        for (uint32_t q = 0; q < TK; ++q) acc += ys[t * TK + q][r];
        if (y_f32) reinterpret_cast<float*>(Y)[(size_t)t * HID + m] = acc;
        else reinterpret_cast<uint16_t*>(Y)[(size_t)t * HID + m] = f2h(acc);
    }
}

// ---------------------------------------------------------------------------
// Streaming gate/up and down (the block's default at every batch whose
// activations fit in LDS): one workgroup per CU, 8 waves, each wave streams
// (expert, row pair) items through a 2-deep ring of register slots, so the
// loads of the next item are in flight while the current one is computed.
// Half-wave 0 takes one row of the pair, half-wave 1 the other; lane c0 of a
// half takes 16-byte chunks c0 + 32j of its row (J chunks). The activations
// (x for gate/up, h for down) are prepared once per workgroup in LDS as
// permuted fp16 pairs with per-chunk (sum, offset constant), so no wave
// repeats that work. Loads are buffer loads on a descriptor over the
// expert's blob: row offsets go in the scalar offset, lane offsets are
// constants, and chunks past the row's end load out of range (zeros, no
// traffic).
// ---------------------------------------------------------------------------
constexpr int kStWaves = 8;
constexpr uint32_t kABlk = 2304;  // per (vector, j): 4 planes x 32 lanes x 16 B + 32 x float2
constexpr int kStXr = 16;         // activation words a thread stages (one pass)
constexpr uint32_t kStOOB = 0x80000000u;

__host__ __device__ inline size_t st_act_bytes(uint32_t nvec, uint32_t K) {
    return (size_t)nvec * (((K >> 5) + 31) / 32) * kABlk;
}

// The J chunks of one row of a projection (as loaded) and its output bias.
template <int J>
struct StSlot {
    u32x4 w[J];
    uint16_t s[J], b[J];  // bf16 bits, widened at use
    uint16_t bi;
};

// Lane-constant offsets into an expert's blob for the row pair's two halves.
template <int J>
struct StLane {
    uint32_t w[J], s[J], b[J], bi;
};

// proj: the half's projection in the blob; rw / rm / rb: the byte distance
// of the half's row from the item's row in W, the metadata and the bias (the
// next row for down, 0 for gate/up).
template <int J>
__device__ __forceinline__ StLane<J> st_lane(uint64_t proj, const kq_moe_desc& d, uint32_t K,
                                             uint32_t rw, uint32_t rm, uint32_t rb) {
    const uint32_t nch = K >> 5, c0 = threadIdx.x & 31;
    StLane<J> o;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t ch = c0 + 32 * j;
        const bool ok = ch < nch;
        o.w[j] = ok ? (uint32_t)(proj + d.sub_w) + rw + ch * 16 : kStOOB;
        o.s[j] = ok ? (uint32_t)(proj + d.sub_s) + rm + (ch >> 1) * 2 : kStOOB;
        o.b[j] = ok ? (uint32_t)(proj + d.sub_b) + rm + (ch >> 1) * 2 : kStOOB;
    }
    o.bi = (uint32_t)(proj + d.sub_bi) + rb;
    return o;
}

// Issue the loads of one row pair: wo = row byte offset in W, mo = row
// offset in the metadata, bo = row offset in the bias (all uniform).
template <int J>
__device__ __forceinline__ void st_issue(StSlot<J>& e, rsrc_t r, const StLane<J>& L, uint32_t wo,
                                         uint32_t mo, uint32_t bo) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        e.w[j] = __builtin_amdgcn_raw_buffer_load_b128(r, L.w[j], wo, kNT);
        e.s[j] = __builtin_amdgcn_raw_buffer_load_b16(r, L.s[j], mo, 0);
        e.b[j] = __builtin_amdgcn_raw_buffer_load_b16(r, L.b[j], mo, 0);
    }
    e.bi = __builtin_amdgcn_raw_buffer_load_b16(r, L.bi, bo, 0);
}

// Activation staging, part 1: every load of nvec fp16 vectors of K elements
// (vector v at src + v * K), issued before the ring so the waits that finish
// the staging never wait for weights. AUX: the loads' cache policy (kCoh:
// device-coherent, for vectors other workgroups of the same launch wrote).
struct StStage {
    u32x4 sv[kStXr];
    uint32_t total;
};
constexpr int kCoh = 16;  // sc1: agent-scope coherent access
template <int AUX = 0>
__device__ __forceinline__ void st_stage_load(StStage& st, const uint16_t* src, uint32_t nvec,
                                              uint32_t K) {
    const uint32_t nthr = blockDim.x, tid = threadIdx.x;
    st.total = nvec * (K >> 3);
    const rsrc_t r = make_rsrc(src, nvec * K * 2);
#pragma unroll
    for (int i = 0; i < kStXr; ++i) {
        if ((uint32_t)i * nthr >= st.total) break;  // uniform
        const uint32_t w = i * nthr + tid;
        st.sv[i] = __builtin_amdgcn_raw_buffer_load_b128(r, w < st.total ? w * 16 : kStOOB, 0, AUX);
    }
}
// Part 2: permuted pairs and chunk constants into the LDS blocks
// [(v * J + j) * kABlk]: planes jw at jw * 512 + c0 * 16, (sum, const) at
// 2048 + c0 * 8; chunks past K are zero. The caller synchronises.
// st_word_store: word w (8 elements) of the staged vectors, every lane of
// the wave taking part (quad sums), the store only if w < total.
// AT: the chunk's sum s comes in sx (the atomic block's sum(h) of the chunk)
// instead of from the staged values; its offset constant still does.
template <int J, bool AT = false>
__device__ __forceinline__ void st_word_store(const u32x4& sv, uint32_t w, uint32_t total,
                                              unsigned char* act, uint32_t nw, float sx = 0.0f) {
    float s, c;
    word_consts(sv, s, c);
    if constexpr (AT) s = sx;
    else s = quad_sum(s);
    c = quad_sum(c);
    if (w < total) {
        const uint32_t v = w / nw, wi = w - v * nw, ch = wi >> 2, jw = wi & 3;
        unsigned char* blk = act + (v * J + (ch >> 5)) * kABlk;
        *reinterpret_cast<u32x4*>(blk + jw * 512 + (ch & 31) * 16) = pair_perm(sv);
        if (jw == 0) *reinterpret_cast<float2*>(blk + 2048 + (ch & 31) * 8) = make_float2(s, c);
    }
}
template <int J>
__device__ __forceinline__ void st_pad_store(unsigned char* act, uint32_t nvec, uint32_t K) {
    const uint32_t nthr = blockDim.x, tid = threadIdx.x, nch = K >> 5;
    const uint32_t npad = 32 * J - nch;
    for (uint32_t i = tid; i < nvec * 5 * npad; i += nthr) {
        const uint32_t v = i / (5 * npad), rem = i - v * 5 * npad, jw = rem / npad;
        const uint32_t ch = nch + (rem - jw * npad);
        unsigned char* blk = act + (v * J + (ch >> 5)) * kABlk;
        if (jw < 4) *reinterpret_cast<u32x4*>(blk + jw * 512 + (ch & 31) * 16) = u32x4{0, 0, 0, 0};
        else *reinterpret_cast<float2*>(blk + 2048 + (ch & 31) * 8) = make_float2(0.0f, 0.0f);
    }
}
template <int J>
__device__ __forceinline__ void st_stage_store(const StStage& st, unsigned char* act, uint32_t nvec,
                                               uint32_t K) {
    const uint32_t nthr = blockDim.x, tid = threadIdx.x, nw = K >> 3;
#pragma unroll
    for (int i = 0; i < kStXr; ++i) {
        if ((uint32_t)i * nthr >= st.total) break;  // uniform
        st_word_store<J>(st.sv[i], i * nthr + tid, st.total, act, nw);
    }
    st_pad_store<J>(act, nvec, K);
}
// The atomic block's chunk sums for the words a thread stages (vector v,
// chunk c at xsh[v * ceil(K / 32) + c]), loaded with the staging loads.
struct StSums {
    float v[kStXr];
};
__device__ __forceinline__ void st_sums_load(StSums& ss, const StStage& st, const float* xsh,
                                             uint32_t K) {
    const uint32_t nthr = blockDim.x, tid = threadIdx.x, nw = K >> 3, nq = (K + 31) >> 5;
#pragma unroll
    for (int i = 0; i < kStXr; ++i) {
        if ((uint32_t)i * nthr >= st.total) break;  // uniform
        const uint32_t w = min(i * nthr + tid, st.total - 1), v = w / nw;
        ss.v[i] = xsh[v * nq + ((w - v * nw) >> 2)];
    }
}
template <int J>
__device__ __forceinline__ void st_stage_store_sums(const StStage& st, const StSums& ss,
                                                    unsigned char* act, uint32_t nvec, uint32_t K) {
    const uint32_t nthr = blockDim.x, tid = threadIdx.x, nw = K >> 3;
#pragma unroll
    for (int i = 0; i < kStXr; ++i) {
        if ((uint32_t)i * nthr >= st.total) break;  // uniform
        st_word_store<J, true>(st.sv[i], i * nthr + tid, st.total, act, nw, ss.v[i]);
    }
    st_pad_store<J>(act, nvec, K);
}

// The dequantised words of one row pair (token-independent).
template <int J>
struct StDq {
    u32x4 d[J][4];
    float sc[J], bs[J];
};
template <int J>
__device__ __forceinline__ void st_dequant(const StSlot<J>& e, const DequantConsts& kc, StDq<J>& q) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        q.d[j][0] = dq4(e.w[j].x, kc);
        q.d[j][1] = dq4(e.w[j].y, kc);
        q.d[j][2] = dq4(e.w[j].z, kc);
        q.d[j][3] = dq4(e.w[j].w, kc);
        q.sc[j] = bf2f(e.s[j]);
        q.bs[j] = bf2f(e.b[j]);
    }
}
// Per-lane partial dot of the row with activation vector v.
template <int J>
__device__ __forceinline__ float st_dot(const StDq<J>& q, const unsigned char* act, uint32_t v) {
    const uint32_t c0 = threadIdx.x & 31;
    const unsigned char* bx = act + v * (J * kABlk) + c0 * 16;
    const unsigned char* bk = act + v * (J * kABlk) + 2048 + c0 * 8;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const u32x4 p0 = *reinterpret_cast<const u32x4*>(bx + j * kABlk);
        const u32x4 p1 = *reinterpret_cast<const u32x4*>(bx + j * kABlk + 512);
        const u32x4 p2 = *reinterpret_cast<const u32x4*>(bx + j * kABlk + 1024);
        const u32x4 p3 = *reinterpret_cast<const u32x4*>(bx + j * kABlk + 1536);
        const float2 k2 = *reinterpret_cast<const float2*>(bk + j * kABlk);
        const float da = dot4(q.d[j][2], p2, dot4(q.d[j][0], p0, 0.0f));
        const float db = dot4(q.d[j][3], p3, dot4(q.d[j][1], p1, 0.0f));
        acc = fmaf(q.sc[j], (da + db) - k2.y, fmaf(q.bs[j], k2.x, acc));
    }
    return acc;
}

// The activation chunks of one vector held in registers (one token).
template <int J>
struct StX {
    u32x4 p[J][4];
    float2 k[J];
};
template <int J>
__device__ __forceinline__ void st_xload(StX<J>& x, const unsigned char* act, uint32_t v) {
    const uint32_t c0 = threadIdx.x & 31;
    const unsigned char* bx = act + v * (J * kABlk) + c0 * 16;
    const unsigned char* bk = act + v * (J * kABlk) + 2048 + c0 * 8;
#pragma unroll
    for (int j = 0; j < J; ++j) {
#pragma unroll
        for (int jw = 0; jw < 4; ++jw) x.p[j][jw] = *reinterpret_cast<const u32x4*>(bx + j * kABlk + jw * 512);
        x.k[j] = *reinterpret_cast<const float2*>(bk + j * kABlk);
    }
}
template <int J>
__device__ __forceinline__ float st_dotx(const StDq<J>& q, const StX<J>& x) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const float da = dot4(q.d[j][2], x.p[j][2], dot4(q.d[j][0], x.p[j][0], 0.0f));
        const float db = dot4(q.d[j][3], x.p[j][3], dot4(q.d[j][1], x.p[j][1], 0.0f));
        acc = fmaf(q.sc[j], (da + db) - x.k[j].y, fmaf(q.bs[j], x.k[j].x, acc));
    }
    return acc;
}

// st_dotx with the dequantisation folded in chunk by chunk (one activation
// vector: the dequantised words are not reused, so they need not all be live).
template <int J>
__device__ __forceinline__ float st_dotx_dq(const StSlot<J>& e, const DequantConsts& kc,
                                            const StX<J>& x) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const u32x4 d0 = dq4(e.w[j].x, kc), d1 = dq4(e.w[j].y, kc);
        const u32x4 d2 = dq4(e.w[j].z, kc), d3 = dq4(e.w[j].w, kc);
        const float da = dot4(d2, x.p[j][2], dot4(d0, x.p[j][0], 0.0f));
        const float db = dot4(d3, x.p[j][3], dot4(d1, x.p[j][1], 0.0f));
        acc = fmaf(bf2f(e.s[j]), (da + db) - x.k[j].y, fmaf(bf2f(e.b[j]), x.k[j].x, acc));
    }
    return acc;
}

// Gate/up: items are (distinct expert u, row i) in u-major order; workgroup
// w takes a contiguous range, wave q every kStWaves-th item of it. Half 0
// reads gate row i, half 1 up row i. XREG (one token): the token's
// activation chunks stay in registers for the whole stream.
// SRC: 0 plan from idx, 1 plan from the router, 2 top-k from the router's
// logits (lg) here, publishing idx / wgt / plan (workgroup 0).
// AT (the atomic sum(h) block, moe-fused/src/kernels.metal:410-451): every h
// value, as a float before its fp16 rounding, is also summed into xsh[slot][row
// / 32] (order-nondeterministic sums): first per workgroup in LDS (ds_add_f32,
// outside the vector-memory counter the ring waits on), then one device-scope
// float atomic per (slot, chunk) the workgroup touched, after its stream. (A
// device atomic per h value, inside the stream, took the block from 21.8 to
// 29.8 us at one token: each one joined the next ring wait.)
template <int J, int SRC, bool XREG, bool AT = false>
__global__ __launch_bounds__(64 * kStWaves) void moe_gu_stream_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx,
    const Plan* __restrict__ plan_g, const uint16_t* __restrict__ xh, uint16_t* __restrict__ H,
    uint32_t batch, const float* __restrict__ lg, uint32_t* __restrict__ idx_out,
    float* __restrict__ wgt_out, Plan* __restrict__ plan_out, float* __restrict__ xsh = nullptr) {
    extern __shared__ __align__(16) unsigned char act[];
    __shared__ Plan ps;
    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    __shared__ uint32_t bits[8];
    __shared__ uint32_t s_next;  // next item of the workgroup's range to hand out
    const uint32_t K = d.hidden, IN = d.inter, TK = d.top_k;
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t half = lane >> 5, rowb = K >> 1, metab = (K >> 6) * 2;

    StStage st;
    st_stage_load(st, xh, batch, K);
    // One token with the top-k here (RP): plan entry u is slot u, so each wave
    // keeps the plan in registers -- lane u holds entry u's expert and weight
    // -- and reads it by readlane: no LDS round trip stands between the logits
    // and the first weight load (the LDS form wrote the picks, read them back,
    // wrote the plan and read it again).
    constexpr bool RP = SRC == 2 && XREG;
    uint32_t rexp = 0, nexp;
    float rwgt = 0.0f;
    if constexpr (RP) {
        const uint32_t NE = d.n_experts;
        float xl[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) xl[q] = lg[min(lane + 64 * q, NE - 1)];
        topk_lanes(xl, NE, TK, rexp, rwgt);
        nexp = TK;
    } else {
        if constexpr (SRC == 2)
            plan_from_logits(lg, batch, d.n_experts, TK, ps, s_idx, s_wgt);
        else
            get_plan<SRC == 1>(plan_g, idx, nullptr, batch * TK, d.n_experts, ps, s_idx, s_wgt, bits);
        nexp = ps.n;
    }
    // expert of plan entry u (uniform)
    auto plan_expert = [&](uint32_t u) __attribute__((always_inline)) {
        const uint32_t uu = min(u, nexp - 1);
        if constexpr (RP) return min((uint32_t)__builtin_amdgcn_readlane((int)rexp, (int)uu), d.n_experts - 1);
        else return (uint32_t)__builtin_amdgcn_readfirstlane(min(ps.expert[uu], d.n_experts - 1));
    };
    const uint32_t N = nexp * IN;
    const uint32_t per = (N + gridDim.x - 1) / gridDim.x, k0 = blockIdx.x * per;
    const uint32_t cnt = k0 < N ? min(per, N - k0) : 0;
    const uint32_t nit = cnt > wave ? (cnt - wave + kStWaves - 1) / kStWaves : 0;
    // AT: the chunks (plan entry u, row / 32) of this workgroup's items are
    // cg0 .. cg0 + nchw - 1 in cg = u * nq + row / 32; lacc[slot][cg - cg0]
    // (LDS after the staged x) sums their h values
    const uint32_t nq = (IN + 31) >> 5, nsl = batch * TK;
    uint32_t cg0 = 0, nchw = 0;
    float* lacc = reinterpret_cast<float*>(act + st_act_bytes(batch, K));
    if constexpr (AT) {
        if (cnt) {
            const uint32_t kb = k0 + cnt - 1;
            cg0 = (k0 / IN) * nq + (k0 % IN) / 32;
            nchw = (kb / IN) * nq + (kb % IN) / 32 - cg0 + 1;
        }
        for (uint32_t i = threadIdx.x; i < nsl * nchw; i += blockDim.x) lacc[i] = 0.0f;
    }

    const StLane<J> L = st_lane<J>(half ? d.off_up : d.off_gate, d, K, 0, 0, 0);
    constexpr int D = 2;
    StSlot<J> ring[D];
    // item cursors (u, i), advanced by kStWaves items without division
    struct Cur {
        uint32_t u, i;
    };
    auto adv = [&](Cur& c) __attribute__((always_inline)) {
        c.i += kStWaves;
        while (c.i >= IN) {  // uniform
            c.i -= IN;
            ++c.u;
        }
    };
    Cur ci{(k0 + wave) / IN, (k0 + wave) % IN}, cc = ci, clast = ci;
    uint32_t nis = 0;  // items issued
    // Item k of the workgroup's range -> (plan entry u, row i): a multiply by
    // 2^32 / IN rounded up, exact here (k0 + k < 2^32 / IN) and checked once.
    const uint32_t inv_in = 0xFFFFFFFFu / IN + 1u;
    auto item = [&](uint32_t k) __attribute__((always_inline)) {
        const uint32_t g = k0 + k;
        uint32_t u = __umulhi(g, inv_in);
        if ((u + 1) * IN <= g) ++u;
        return Cur{u, g - u * IN};
    };
    // Without AT, the items past each wave's first D go out one at a time to
    // whichever wave refills a slot first (an LDS counter): the older wave of
    // a SIMD issues ahead of the younger, and a fixed deal (items wave,
    // wave + 8, ...) left the younger waves ~0.5-0.8 us behind at the end.
    // An item past the range loads through an empty descriptor (no traffic,
    // the same load count).
    auto issue_k = [&](StSlot<J>& e, uint32_t k) __attribute__((always_inline)) {
        const bool ok = k < cnt;  // uniform
        const Cur c = item(ok ? k : 0);
        const uint32_t ex = plan_expert(c.u);
        const rsrc_t r = make_rsrc(pool + (size_t)ex * d.blob, ok ? (uint32_t)d.blob : 0u);
        const uint32_t i = __builtin_amdgcn_readfirstlane(c.i);
        st_issue<J>(e, r, L, i * rowb, i * metab, i * 2);
    };
    uint32_t sk[D];  // the item each ring slot holds (dynamic hand-out)
    auto issue = [&](StSlot<J>& e) __attribute__((always_inline)) {
        if (nis < nit) clast = ci;  // padding re-reads the last item
        const uint32_t ex = plan_expert(clast.u);
        const rsrc_t r = make_rsrc(pool + (size_t)ex * d.blob, (uint32_t)d.blob);
        const uint32_t i = __builtin_amdgcn_readfirstlane(clast.i);
        st_issue<J>(e, r, L, i * rowb, i * metab, i * 2);
        adv(ci);
        ++nis;
    };
    // primed even without items (a valid row, unused): the same number of
    // loads on every path lets the compiler wait for the staging loads alone
#pragma unroll
    for (int s = 0; s < D; ++s) {
        if constexpr (AT) {
            issue(ring[s]);
        } else {
            sk[s] = wave + s * kStWaves;
            issue_k(ring[s], sk[s]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (!AT && threadIdx.x == 0) s_next = D * kStWaves;
    if constexpr (RP) {  // what publish_plan writes, from the registers
        if (blockIdx.x == 0 && wave == 0) {
            if (lane < TK) {
                idx_out[lane] = rexp;
                wgt_out[lane] = rwgt;
                plan_out->expert[lane] = min(rexp, d.n_experts - 1);
                plan_out->mask[lane][0] = 1ull << lane;
                plan_out->mask[lane][1] = 0;
            }
            if (lane == 0) plan_out->n = TK;
        }
    } else if constexpr (SRC == 2) {
        if (blockIdx.x == 0) publish_plan(ps, s_idx, s_wgt, batch * TK, idx_out, wgt_out, plan_out);
    }
    st_stage_store<J>(st, act, batch, K);
    __syncthreads();
    if (nit == 0) return;
    StX<J> xr;
    if constexpr (XREG) st_xload<J>(xr, act, 0);

    const DequantConsts kc;
    // One store per step, by every lane: lane j < the item's slot count writes
    // slot j's h, the other lanes repeat the last slot's write. A fixed store
    // count keeps the next ring wait from also waiting for this step's store.
    // Steps of the main loop are never padding; only the tail checks. `mid`
    // runs between the step's plan reads and its first use of the weights.
    auto step = [&](const StSlot<J>& e, uint32_t it, bool tail, auto&& mid) __attribute__((always_inline)) {
        if (tail && it >= nit) return;  // padding (uniform)
        uint64_t m0, m1;
        if constexpr (RP) {
            m0 = 1ull << cc.u;
            m1 = 0;
        } else {
            m0 = ps.mask[cc.u][0];
            m1 = ps.mask[cc.u][1];
        }
        mid();
        StDq<J> q;
        st_dequant<J>(e, kc, q);
        const float bg = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 0));
        const float bu = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 32));
        size_t oi = 0;
        uint16_t ov = 0;
        for (uint32_t k = 0; m0 | m1; ++k) {
            const uint32_t s = pop_slot(m0, m1);
            float acc;
            if constexpr (XREG) acc = st_dotx<J>(q, xr);
            else acc = st_dot<J>(q, act, s / TK);
            const float2 hs = half_sums(acc);
            const float hf = swiglu(hs.x + bg, hs.y + bu);
            const uint16_t hv = f2h(hf);
            if constexpr (AT) {
                if (lane == 0)
                    __hip_atomic_fetch_add(lacc + s * nchw + (cc.u * nq + (cc.i >> 5) - cg0), hf,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            if (lane >= k) {
                oi = (size_t)s * IN + cc.i;
                ov = hv;
            }
        }
        H[oi] = ov;
        adv(cc);
    };
    if constexpr (!AT) {
        // items in increasing order per wave: the first slot that holds an
        // item past the range ends the wave's stream
        auto step_k = [&](const StSlot<J>& e, uint32_t k, auto&& mid) __attribute__((always_inline)) {
            cc = item(k);
            step(e, 0, false, mid);
        };
        // The next index: an LDS atomic by lane 0 alone, with the exec mask
        // narrowed and restored inside one asm block (a one-lane atomic
        // written as a branch left the waitcnt pass waiting for every load at
        // the loop head; all 64 lanes on the one address serialise in LDS).
        // The same block waits for the return (the compiler does not see
        // that wait, so a return left in flight in a register past the asm
        // could be copied before it arrives); lane 0's value is then made
        // uniform outside it (an asm with a VGPR output counts as divergent).
        // Each step draws after its plan reads, before it waits for its
        // weights (far longer than an LDS atomic), and refills its slot with
        // the drawn item.
        const uint32_t next_a =
            (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_next;
        auto draw = [&]() __attribute__((always_inline)) {
            uint32_t v;
            uint64_t saved;
            asm volatile(
                "s_mov_b64 %1, exec\n\t"
                "s_mov_b64 exec, 1\n\t"
                "ds_add_rtn_u32 %0, %2, %3\n\t"
                "s_mov_b64 exec, %1\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(v), "=&s"(saved)
                : "v"(next_a), "v"(1u)
                : "memory");
            return __builtin_amdgcn_readfirstlane(v);
        };
        // every step refills its slot (an item past the range moves no
        // bytes), so the loop body has one path and each wait counts exactly
        // the other slot's loads and the step's store
        static_assert(D == 2, "the loop body is written for two slots");
        auto run = [&](int s) __attribute__((always_inline)) {
            uint32_t nk = 0;
            step_k(ring[s], sk[s], [&]() __attribute__((always_inline)) {
                __builtin_amdgcn_sched_barrier(0);
                nk = draw();
                __builtin_amdgcn_sched_barrier(0);
            });
            __builtin_amdgcn_sched_barrier(0);
            sk[s] = nk;
            issue_k(ring[s], sk[s]);
            __builtin_amdgcn_sched_barrier(0);
        };
        for (;;) {
            if (sk[0] >= cnt) break;  // uniform
            run(0);
            if (sk[1] >= cnt) break;
            run(1);
        }
        return;
    }
    const uint32_t nsteps = (nit + D - 1) / D * D;
    uint32_t it = 0;
    for (; it + D < nsteps; it += D) {
#pragma unroll
        for (int s = 0; s < D; ++s) {
            step(ring[s], it + s, false, [] {});
            issue(ring[s]);
        }
    }
#pragma unroll
    for (int s = 0; s < D; ++s) step(ring[s], it + s, true, [] {});
    if constexpr (AT) {  // every wave's LDS sums done; waves without items (wave >= cnt) have left
        __syncthreads();
        const uint32_t nact = 64 * min(cnt, (uint32_t)kStWaves);
        for (uint32_t i = threadIdx.x; i < nsl * nchw; i += nact) {
            const float v = lacc[i];
            const uint32_t sl = i / nchw, cg = cg0 + (i - sl * nchw);
            if (v != 0.0f)  // only (slot, chunk) pairs of this workgroup's items hold sums
                __hip_atomic_fetch_add(xsh + (size_t)sl * nq + cg % nq, v, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Down + weighted combine: workgroup w owns output row pairs [p0, p1) for
// every distinct expert; items are (u, pair) in u-major order. Per-slot
// wgt * (down . h + bias) goes to LDS and the slots are summed in k order
// after the stream (deterministic, no atomics).
// AT (the atomic sum(h) block, moe-fused/src/kernels.metal:453-487): the
// chunk sums of h come from xsh, which the gate/up launch accumulated.
template <int J, bool FROM_PLAN, bool AT = false>
__global__ __launch_bounds__(64 * kStWaves) void moe_dn_stream_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint32_t* __restrict__ idx,
    const float* __restrict__ wgt, const Plan* __restrict__ plan_g,
    const uint16_t* __restrict__ H, void* __restrict__ Y, int y_f32, uint32_t batch, uint32_t pp,
    const float* __restrict__ xsh = nullptr) {
    extern __shared__ __align__(16) unsigned char act[];  // [nslots h blocks][ys]
    __shared__ Plan ps;
    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    __shared__ uint32_t bits[8];
    const uint32_t HID = d.hidden, K = d.inter, TK = d.top_k, nslots = batch * TK;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t half = lane >> 5, rowb = K >> 1, metab = (K >> 6) * 2;
    float* ys = reinterpret_cast<float*>(act + st_act_bytes(nslots, K));  // [nslots][2 * pp]

    StStage st;
    st_stage_load(st, H, nslots, K);
    StSums ss;
    if constexpr (AT) st_sums_load(ss, st, xsh, K);
    // From the workspace plan, every wave reads the plan and the weights
    // itself at uniform addresses (scalar loads): no LDS copy and no barrier,
    // so the h staging loads stay in flight while the ring is primed.
    if constexpr (!FROM_PLAN)
        get_plan<false>(plan_g, idx, wgt, nslots, d.n_experts, ps, s_idx, s_wgt, bits);
    auto p_expert = [&](uint32_t u) __attribute__((always_inline)) {
        if constexpr (FROM_PLAN) return plan_g->expert[u];
        else return ps.expert[u];
    };
    auto p_mask = [&](uint32_t u, int h) __attribute__((always_inline)) {
        if constexpr (FROM_PLAN) return plan_g->mask[u][h] & slot_bits(nslots, h);
        else return ps.mask[u][h];
    };
    auto p_wgt = [&](uint32_t sl) __attribute__((always_inline)) {
        if constexpr (FROM_PLAN) return wgt[sl];
        else return s_wgt[sl];
    };
    // at most one plan entry per slot; with the masks above, every plan read
    // and every slot index stays within this call's nslots slots
    const uint32_t nexp = min(FROM_PLAN ? plan_g->n : ps.n, nslots), npairs = HID >> 1;
    const uint32_t p0 = blockIdx.x * pp, np = p0 < npairs ? min(pp, npairs - p0) : 0;
    const uint32_t N = nexp * np;
    const uint32_t nit = N > wave ? (N - wave + kStWaves - 1) / kStWaves : 0;

    const StLane<J> L = st_lane<J>(d.off_down, d, K, half * rowb, half * metab, half * 2);
    // ring depth 2: a 3-deep ring (every item of a wave in flight at one
    // token) measured 21.8 -> 22.4 us per block, and a workgroup barrier
    // putting every wave's h loads ahead of all weight loads changed nothing
    constexpr int D = 2;
    StSlot<J> ring[D];
    // item cursors (u, pair), advanced by kStWaves items without division
    struct Cur {
        uint32_t u, p;
    };
    auto adv = [&](Cur& c) __attribute__((always_inline)) {
        c.p += kStWaves;
        while (c.p >= p0 + np) {  // uniform
            c.p -= np;
            ++c.u;
        }
    };
    Cur ci{np ? wave / np : 0, np ? p0 + wave % np : p0}, cc = ci, clast = ci;
    uint32_t nis = 0;  // items issued
    auto issue = [&](StSlot<J>& e) __attribute__((always_inline)) {
        if (nis < nit) clast = ci;  // padding re-reads the last item
        const uint32_t ex =
            __builtin_amdgcn_readfirstlane(min(p_expert(min(clast.u, nexp - 1)), d.n_experts - 1));
        const rsrc_t r = make_rsrc(pool + (size_t)ex * d.blob, (uint32_t)d.blob);
        const uint32_t p = __builtin_amdgcn_readfirstlane(clast.p);
        st_issue<J>(e, r, L, 2 * p * rowb, 2 * p * metab, 2 * p * 2);
        adv(ci);
        ++nis;
    };
    // primed even without items (a valid row pair, unused): the same number
    // of loads on every path lets the compiler wait for the staging loads alone
#pragma unroll
    for (int s = 0; s < D; ++s) {
        issue(ring[s]);
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (AT) st_stage_store_sums<J>(st, ss, act, nslots, K);
    else st_stage_store<J>(st, act, nslots, K);
    __syncthreads();

    const DequantConsts kc;
    auto step = [&](const StSlot<J>& e, uint32_t it) __attribute__((always_inline)) {
        if (it >= nit) return;  // padding (uniform)
        const Cur c = cc;
        adv(cc);
        uint64_t m0 = p_mask(c.u, 0), m1 = p_mask(c.u, 1);
        StDq<J> q;
        st_dequant<J>(e, kc, q);
        const float b0 = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 0));
        const float b1 = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 32));
        const uint32_t r = 2 * (c.p - p0);
        while (m0 | m1) {
            const uint32_t s = pop_slot(m0, m1);
            const float2 hs = half_sums(st_dot<J>(q, act, s));
            const float wt = p_wgt(s);
            if (lane == 0) {
                ys[s * 2 * pp + r] = wt * (hs.x + b0);
                ys[s * 2 * pp + r + 1] = wt * (hs.y + b1);
            }
        }
    };
    if (nit > 0) {
        const uint32_t nsteps = (nit + D - 1) / D * D;
        uint32_t it = 0;
        for (; it + D < nsteps; it += D) {
#pragma unroll
            for (int s = 0; s < D; ++s) {
                step(ring[s], it + s);
                issue(ring[s]);
            }
        }
#pragma unroll
        for (int s = 0; s < D; ++s) step(ring[s], it + s);
    }
    __syncthreads();
    // combine in slot order (moe-fused/src/kernels.metal:254-263)
    for (uint32_t i = tid; i < batch * 2 * np; i += blockDim.x) {
        const uint32_t t = i / (2 * np), r = i - t * 2 * np, m = 2 * p0 + r;
        float acc = 0.0f;
        for (uint32_t q = 0; q < TK; ++q) acc += ys[(t * TK + q) * 2 * pp + r];
        if (y_f32) reinterpret_cast<float*>(Y)[(size_t)t * HID + m] = acc;
        else reinterpret_cast<uint16_t*>(Y)[(size_t)t * HID + m] = f2h(acc);
    }
}

// One-round expert partition (the block's gate/up and down from 3 tokens):
// G workgroups, one per CU; expert u of the plan gets a share of them in
// proportion to its cost, rows * (kPartRow + kPartSlot * slots of u) -- a
// row's weight bytes plus one dot product per slot that chose the expert,
// so experts picked by several tokens get more workgroups (at least one
// each) -- and splits its nrows rows (gate/up rows or down row pairs)
// evenly among them. Workgroup b's expert u starts at
// start(u) = u + floor((G - n) * C_u / W), C_u the cost of the experts
// before u, W the total. Each wave computes the assignment itself: lane l
// loads plan entries l and l + 64 with vector loads (one round trip), a
// wave prefix sum gives every C_u, a ballot finds b's entry, and its expert
// and slot masks come back by readlane.
// Costs: a row's weights 4, each slot's dot product 5 (a two-slot row 1.56x a
// one-slot row). Swept with the 3-deep ring, slot weight 2 / 3 / 4 / 5 / 8 /
// 11 against row weight 4: 4 tokens 52.5 / 52.2 / 51.9 / 51.5 / 51.6 / 51.8,
// 8 tokens 93.7 / 89.4 / 88.5 / 88.5 / 89.1 / 89.3, 16 tokens 174.9 / 163.9 /
// 159.7 / 158.8 / 158.7 / 158.6 us per block.
// Ring depth 3 (long per-wave streams here, ~40 items): against depth 4, 4 / 8 / 16 tokens 53.9 / 92.8 / 166.0 ->
// 52.2 / 89.4 / 163.1 us per block (depth 4 held the one-slot gate/up at
// 256 VGPRs with 3 spilled; depth 2: 51.3 / 89.9 / 166.1).
constexpr uint32_t kPartRow = 4, kPartSlot = 5;
// The gate/up's split (3-7 tokens) prices rows by the form that computes them:
// a workgroup whose one entry is chosen by one slot keeps that token's x in
// registers, faster than the LDS form of the other workgroups. Measured per
// item at 8 tokens (us x workgroups): one slot 0.129 in registers / 0.151
// from LDS, two slots 0.229, three 0.308, i.e. 36 for a one-slot row and
// 21 + 22 s otherwise. Against 4 + 5 s for every row, A/B per block: 3 / 4 /
// 5 / 6 tokens 42.96 / 51.85 / 60.98 / 69.56 -> 42.45 / 51.49 / 60.28 /
// 68.58 us, outputs bitwise equal. (The equal-cost ranges from 8 tokens keep
// 4 + 5 s: a workgroup whose range spans two one-slot entries runs the LDS
// form, and the new prices then left those ~7 us behind.)
constexpr uint32_t kGuOne = 36, kGuRow = 21, kGuSlot = 22;
constexpr int kPartD = 3;
struct PartAssign {
    uint32_t u, r0, nr, ex;  // u = 0xFFFFFFFF: no work for this workgroup
    uint64_t m0, m1;
};
// Inclusive wave64 prefix sum in DPP moves (no LDS round trips): shifts
// right by 1, 2, 4 and 8 within each 16-lane row (lanes with no source add
// 0), then each row's last lane broadcast into the next row (row_bcast:15,
// rows 1 and 3) and lane 31 into rows 2 and 3 (row_bcast:31).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_add(uint32_t v) {
    return v + (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
}
__device__ __forceinline__ uint32_t wave_scan_incl(uint32_t v) {
    v = dpp_add<0x111, 0xf>(v);  // row_shr:1
    v = dpp_add<0x112, 0xf>(v);  // row_shr:2
    v = dpp_add<0x114, 0xf>(v);  // row_shr:4
    v = dpp_add<0x118, 0xf>(v);  // row_shr:8
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31
    return v;
}
__device__ __forceinline__ uint32_t rl(uint32_t v, uint32_t l) {
    return __builtin_amdgcn_readlane(v, l);
}
__device__ __forceinline__ uint64_t rl64(uint64_t v, uint32_t l) {
    return (uint64_t)rl((uint32_t)v, l) | ((uint64_t)rl((uint32_t)(v >> 32), l) << 32);
}
__device__ __forceinline__ PartAssign part_assign(const Plan* plan_g, uint32_t nslots, uint32_t nrows,
                                                  uint32_t n_experts, uint32_t c_one = kPartRow + kPartSlot,
                                                  uint32_t c_row = kPartRow, uint32_t c_slot = kPartSlot) {
    const uint32_t lane = threadIdx.x & 63, G = gridDim.x, b = blockIdx.x;
    const uint64_t sb0 = slot_bits(nslots, 0), sb1 = slot_bits(nslots, 1);
    // every entry's loads first (entries past n are read but unused)
    uint64_t m0[2], m1[2];
    uint32_t ex[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t u = lane + 64 * q;
        m0[q] = plan_g->mask[u][0] & sb0;
        m1[q] = plan_g->mask[u][1] & sb1;
        ex[q] = min(plan_g->expert[u], n_experts - 1);
    }
    const uint32_t n = min(plan_g->n, nslots);
    PartAssign a{0xFFFFFFFFu, 0, 0, 0, 0, 0};
    if (n == 0 || G < n) return a;
    uint32_t c[2], sc[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t sl = (uint32_t)(__popcll(m0[q]) + __popcll(m1[q]));
        c[q] = lane + 64 * q < n ? (sl == 1 ? c_one : c_row + c_slot * sl) : 0u;
    }
    sc[0] = wave_scan_incl(c[0]);
    const uint32_t tot0 = rl(sc[0], 63);
    sc[1] = wave_scan_incl(c[1]) + tot0;
    const uint32_t W = rl(sc[1], 63), spare = G - n;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t u = lane + 64 * q;
        const uint32_t start = u + spare * (sc[q] - c[q]) / W, next = u + 1 + spare * sc[q] / W;
        const uint64_t hit = __ballot(u < n && start <= b && b < next);
        if (hit) {  // uniform
            const uint32_t l = (uint32_t)__builtin_ctzll(hit);
            const uint32_t st = rl(start, l), nu = rl(next, l) - st, cb = b - st;
            a.u = l + 64 * q;
            a.r0 = cb * nrows / nu;
            a.nr = (cb + 1) * nrows / nu - a.r0;
            a.ex = rl(ex[q], l);
            a.m0 = rl64(m0[q], l);
            a.m1 = rl64(m1[q], l);
            return a;
        }
    }
    return a;
}

// Cost-weighted contiguous ranges (the partitioned gate/up): the plan
// entries' rows in entry-major order form one sequence of n * nrows items,
// item (u, i) costing kPartRow + kPartSlot * (slots of u); workgroup b takes
// the items whose cost falls in [b W / G, (b + 1) W / G), W the total, so
// every workgroup gets the same cost to within one row, whatever the number
// of workgroups per entry (a range may span entries). Each wave computes it:
// lanes l and l + 64 hold entries l and l + 64, a wave prefix sum gives each
// entry's first cost, a ballot finds the entry a boundary falls in. Returns
// the range's first item (u * nrows + i) and its item count.
struct PartRange {
    uint32_t g0, n;
};
constexpr uint32_t kPartRangeMin = 8;  // tokens from which the gate/up takes equal-cost ranges
__device__ __forceinline__ uint32_t range_pos(uint32_t X, const uint32_t (&c)[2],
                                              const uint32_t (&cu)[2], uint32_t nrows, uint32_t n) {
    const uint32_t lane = threadIdx.x & 63;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t u = lane + 64 * q;
        const uint32_t lo = cu[q], hi = cu[q] + nrows * c[q];
        const uint64_t hit = __ballot(u < n && c[q] > 0 && lo <= X && X < hi);
        if (hit) {  // uniform
            const uint32_t l = (uint32_t)__builtin_ctzll(hit);
            const uint32_t cl = rl(c[q], l), base = rl(cu[q], l);
            const uint32_t r = (X - base + cl - 1) / cl;  // first row starting at or after X
            return (l + 64 * q) * nrows + r;                         // r == nrows: the next entry's row 0
        }
    }
    return n * nrows;  // X at or past the total
}
__device__ __forceinline__ PartRange part_range(const Plan& ps, uint32_t nslots, uint32_t nrows) {
    const uint32_t lane = threadIdx.x & 63, G = gridDim.x, b = blockIdx.x;
    const uint32_t n = min(ps.n, nslots);
    uint32_t c[2], cu[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint32_t u = lane + 64 * q;
        const uint32_t sl = u < n ? (uint32_t)(__popcll(ps.mask[u][0]) + __popcll(ps.mask[u][1])) : 0u;
        c[q] = u < n ? kPartRow + kPartSlot * sl : 0u;
    }
    // exclusive prefix of the entries' total costs (nrows * c); fits 32 bits:
    // nrows <= 4096, c <= 4 + 5 * 128, n <= 128
    const uint32_t i0 = wave_scan_incl(nrows * c[0]);
    const uint32_t tot0 = rl(i0, 63);
    const uint32_t i1 = wave_scan_incl(nrows * c[1]) + tot0;
    cu[0] = i0 - nrows * c[0];
    cu[1] = i1 - nrows * c[1];
    // the boundaries floor(W b / G) in 32 bits: (W / G) b + (W % G) b / G
    // (32-bit arithmetic: the 64-bit divisions cost ~0.26 us of the prologue)
    const uint32_t W = rl(i1, 63), Wq = W / G, Wr = W - Wq * G;
    const uint32_t s = range_pos(Wq * b + Wr * b / G, c, cu, nrows, n);
    const uint32_t e = range_pos(Wq * (b + 1) + Wr * (b + 1) / G, c, cu, nrows, n);
    return PartRange{s, e - s};
}

// Gate/up + SwiGLU, partitioned by expert (3-16 tokens): workgroup b
// streams the row chunk part_assign gives it of one plan entry's expert
// (half 0 the gate row, half 1 the up row) with only the x vectors of that
// expert's tokens in LDS, and writes h for each of its slots. Each expert's
// rows are read once for all its slots, as in the other forms. One round of
// one workgroup per CU with cost-weighted chunks replaced two rounds of
// equal chunks (two workgroups per CU's worth, which ran as two rounds at
// this register use): 8 tokens 110.6 -> 98.8 us per block with the down
// kernel done the same way.
// The routing comes from the router's logits lg ([batch][n_experts], a
// logits-only router launch before this one): every workgroup runs the
// top-k of every token (wave w takes tokens w, w + 8) and builds the plan in
// LDS; workgroup 0 publishes idx, wgt and the plan for the down launch.
// Every token's x is loaded at entry, right after the wave's logits, and
// staged in LDS by token, so the staging never waits behind the weight ring.
template <int J>
__global__ __launch_bounds__(64 * kStWaves) void moe_gu_part_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const uint16_t* __restrict__ xh,
    uint32_t batch, uint16_t* __restrict__ H, const float* __restrict__ lg,
    uint32_t* __restrict__ idx_out, float* __restrict__ wgt_out, Plan* __restrict__ plan_out) {
    extern __shared__ __align__(16) unsigned char act[];  // [batch x blocks], by token
    __shared__ Plan ps;
    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    __shared__ uint32_t bits[8];
    __shared__ uint32_t s_next;  // next item of the workgroup's range to hand out
    const uint32_t K = d.hidden, IN = d.inter, TK = d.top_k;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t half = lane >> 5, rowb = K >> 1, metab = (K >> 6) * 2;

    // 1. the logits of the wave's tokens (t = wave, wave + 8), then every
    // token's x (K <= 4096, batch <= 16: at most kStXr words per thread). The
    // logits go first, so the top-k waits for them alone (loads retire in
    // order) and not for the x of every token; every wave loads both sets
    // (clamped to a valid token), so the wait counts are exact.
    const uint32_t NE = d.n_experts;
    float lgv[2][4];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t t = min(wave + r * kStWaves, batch - 1);
#pragma unroll
        for (int q = 0; q < 4; ++q) lgv[r][q] = lg[(size_t)t * NE + min(lane + 64 * q, NE - 1)];
    }
    StStage st;
    st_stage_load(st, xh, batch, K);
    // 2. top-k of every token, then the plan
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const uint32_t t = wave + r * kStWaves;
        if (t < batch) topk_vals(lgv[r], NE, TK, s_idx + t * TK, s_wgt + t * TK);  // uniform
    }
    __syncthreads();
    build_plan(s_idx, batch * TK, d.n_experts, ps, bits);
    if (blockIdx.x == 0) publish_plan(ps, s_idx, s_wgt, batch * TK, idx_out, wgt_out, plan_out);
    // 3. this workgroup's range of (plan entry u, row i) items, u-major: from
    // 8 tokens equal-cost ranges (a range may span entries), below that the
    // whole-workgroup split of part_assign (one entry per workgroup, so every
    // one-slot workgroup holds x in registers). Measured per block against
    // part_assign at every batch: 3 / 4 tokens 42.7 / 52.0 us against 43.8 /
    // 52.6 with ranges, 8 / 16 tokens 90.0 / 157.6 against 89.4 / 155.2.
    PartRange pr{0, 0};
    if (batch >= kPartRangeMin) {
        pr = part_range(ps, batch * TK, IN);
    } else {
        const PartAssign pa = part_assign(&ps, batch * TK, IN, d.n_experts, kGuOne, kGuRow, kGuSlot);
        if (pa.u != 0xFFFFFFFFu) pr = PartRange{pa.u * IN + pa.r0, pa.nr};
    }
    const uint32_t N = pr.n;
    const uint32_t nexp = min(ps.n, batch * TK);
    if (nexp == 0) return;  // uniform (never: every token selects top_k experts)
    struct Cur {
        uint32_t u, i;
    };
    // Item k of the workgroup's range -> (plan entry u, row i): a multiply by
    // 2^32 / IN rounded up, exact here (pr.g0 + k < 2^32 / IN) and checked once.
    const uint32_t inv_in = 0xFFFFFFFFu / IN + 1u;
    auto item = [&](uint32_t k) __attribute__((always_inline)) {
        const uint32_t g = pr.g0 + k;
        uint32_t u = __umulhi(g, inv_in);
        if ((u + 1) * IN <= g) ++u;
        return Cur{u, g - u * IN};
    };

    // 4. prime the ring: a wave's first D items are items wave, wave + 8, ...;
    // every later one goes out through an LDS counter to whichever wave
    // refills a slot first (the SIMDs issue for their older waves first, and
    // a fixed deal left the younger waves behind at the end). An item past
    // the range loads through an empty descriptor (no traffic, the same load
    // count).
    const StLane<J> L = st_lane<J>(half ? d.off_up : d.off_gate, d, K, 0, 0, 0);
    constexpr int D = kPartD;
    static_assert(D == 3, "the loop body is written for three slots");
    auto issue_k = [&](StSlot<J>& e, uint32_t k) __attribute__((always_inline)) {
        const bool ok = k < N;  // uniform
        const Cur c = item(ok ? k : 0);
        const uint32_t ex = __builtin_amdgcn_readfirstlane(
            min(ps.expert[min(c.u, nexp - 1)], d.n_experts - 1));
        const rsrc_t r = make_rsrc(pool + (size_t)ex * d.blob, ok ? (uint32_t)d.blob : 0u);
        const uint32_t i = __builtin_amdgcn_readfirstlane(min(c.i, IN - 1));
        st_issue<J>(e, r, L, i * rowb, i * metab, i * 2);
    };

    // 5, 6. prime the ring, store the staged x (vector = token, chunks past
    // K zero), then stream. Each form below primes its own ring (one primed
    // before the choice left the other copying its registers, and so waiting
    // for every load, at its loop head); the choice is uniform in the
    // workgroup, so the barrier inside it is too.
    const DequantConsts kc;
    // One store per step by every lane (lane j < the item's slot count: slot
    // j; the rest repeat the last), so the next ring wait does not also wait
    // for it; only the tail checks for padding. XR (the whole range in one
    // entry chosen by one slot, the common case): the token's x chunks are
    // held in registers, so the loop reads no LDS.
    const uint32_t ua = pr.g0 / IN, ub = (pr.g0 + N - 1) / IN;
    // The draw: an LDS atomic by lane 0 alone, exec narrowed and restored
    // inside one asm block that also waits for the return (a one-lane atomic
    // written as a branch left the waitcnt pass waiting for every load at
    // the loop head; a return left in flight in a register past the asm could
    // be copied before it arrives); lane 0's value is made uniform outside it.
    const uint32_t next_a =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_next;
    auto draw = [&]() __attribute__((always_inline)) {
        uint32_t v;
        uint64_t saved;
        asm volatile(
            "s_mov_b64 %1, exec\n\t"
            "s_mov_b64 exec, 1\n\t"
            "ds_add_rtn_u32 %0, %2, %3\n\t"
            "s_mov_b64 exec, %1\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v), "=&s"(saved)
            : "v"(next_a), "v"(1u)
            : "memory");
        return __builtin_amdgcn_readfirstlane(v);
    };
    auto run = [&](auto xr_tag) __attribute__((always_inline)) {
        constexpr bool XR = decltype(xr_tag)::value;
        StSlot<J> ring[D];
        uint32_t sk[D];  // the item each ring slot holds
#pragma unroll
        for (int q = 0; q < D; ++q) {
            sk[q] = wave + q * kStWaves;
            issue_k(ring[q], sk[q]);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (threadIdx.x == 0) s_next = D * kStWaves;
        st_stage_store<J>(st, act, batch, K);
        __syncthreads();
        if (wave >= N) return;  // no items; no later barrier
        StX<J> xr;
        if constexpr (XR) {
            uint64_t ma = ps.mask[ua][0], mb = ps.mask[ua][1];
            st_xload<J>(xr, act, pop_slot(ma, mb) / TK);
        }
        // a step draws the item its slot takes next between its plan read
        // and its first use of the weights (far longer than an LDS atomic)
        auto step = [&](const StSlot<J>& e, const Cur c, uint32_t& nk) __attribute__((always_inline)) {
            uint64_t ma = ps.mask[c.u][0], mb = ps.mask[c.u][1];
            __builtin_amdgcn_sched_barrier(0);
            nk = draw();
            __builtin_amdgcn_sched_barrier(0);
            StDq<J> q;
            if constexpr (!XR) st_dequant<J>(e, kc, q);
            const float bg = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 0));
            const float bu = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 32));
            const uint32_t nv = XR ? 1u : (uint32_t)(__popcll(ma) + __popcll(mb));
            size_t oi = 0;
            uint16_t ov = 0;
            for (uint32_t k = 0; k < nv; ++k) {
                const uint32_t sl = pop_slot(ma, mb);
                float acc;
                if constexpr (XR) acc = st_dotx_dq<J>(e, kc, xr);
                else acc = st_dot<J>(q, act, sl / TK);
                const float2 hs = half_sums(acc);
                const uint16_t hv = f2h(swiglu(hs.x + bg, hs.y + bu));
                if (lane >= k) {
                    oi = (size_t)sl * IN + c.i;
                    ov = hv;
                }
            }
            H[oi] = ov;
        };
        // every step refills its slot (an item past the range moves no
        // bytes), so the loop body has one path; a wave's items only grow,
        // so the first slot past the range ends its stream
        // a slot past the range stores once through an empty descriptor
        // (dropped) and refills out of range, so every path through the loop
        // issues the same stores and loads and each wait counts exactly the
        // other slots'
        const rsrc_t rnull = make_rsrc(H, 0);
        auto slot = [&](int s, bool live) __attribute__((always_inline)) {
            uint32_t nk = N;
            if (live) step(ring[s], item(sk[s]), nk);  // uniform
            else __builtin_amdgcn_raw_buffer_store_b16((uint16_t)0, rnull, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            sk[s] = nk;
            issue_k(ring[s], nk);
            __builtin_amdgcn_sched_barrier(0);
        };
        // One exit, at the top: with an exit after each slot the compiler
        // sank a slot's refill loads past the next exit test (they are dead
        // on that path) and past the next slot's work. A slot past the range
        // means every later slot is, and so is the refilled slot 0.
        while (sk[0] < N) {  // uniform
            slot(0, true);
            slot(1, sk[1] < N);
            slot(2, sk[2] < N);
        }
    };
    // (at J = 4 the registers of the one-slot form would spill)
    const bool one = ua == ub && __popcll(ps.mask[ua][0]) + __popcll(ps.mask[ua][1]) == 1;
    if (J <= 3 && one) run(std::integral_constant<bool, J <= 3>{});  // uniform
    else run(std::false_type{});
}

// Down + weighted products, partitioned by expert (from 6 tokens, where the
// slots' h vectors no longer fit one workgroup's LDS): workgroup b streams
// the row-pair chunk part_assign gives it of one plan entry's expert with
// only that expert's h vectors in LDS (one per slot that chose it, at most
// one per token), and writes wgt_s * (down . h_s + bias) for each of those
// slots s to ys[s][*]. moe_combine_k then sums each token's slots in k
// order, as the reference's combine does (moe-fused/src/kernels.metal:254-263).
// (Combining in the last workgroup of each row chunk instead measured slower:
// 125 us per block at 8 tokens with device-coherent stores, 130 with fences,
// against 119 with the separate launch.)
template <int J>
__global__ __launch_bounds__(64 * kStWaves) void moe_dn_part_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const float* __restrict__ wgt,
    const Plan* __restrict__ plan_g, const uint16_t* __restrict__ H, uint32_t nslots,
    float* __restrict__ ys) {
    extern __shared__ __align__(16) unsigned char act[];  // [nvec h blocks]
    __shared__ uint32_t s_next;  // next row pair of the workgroup's range to hand out
    const uint32_t HID = d.hidden, K = d.inter, nw = K >> 3, nch = K >> 5;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t half = lane >> 5, rowb = K >> 1, metab = (K >> 6) * 2;
    const PartAssign pa = part_assign(plan_g, nslots, HID >> 1, d.n_experts);
    if (pa.u == 0xFFFFFFFFu) return;  // uniform: no share of the plan
    const uint32_t ex = pa.ex;
    const uint64_t mk0 = pa.m0, mk1 = pa.m1;
    const uint32_t nvec = __popcll(mk0) + __popcll(mk1);
    const uint32_t p0 = pa.r0, np = pa.nr;

    // 1. the expert's h vectors, slot order: word tid of vector k (K <= 4096: nw <= threads)
    const rsrc_t rh = make_rsrc(H, nslots * K * 2);
    u32x4 sv[kStXr];
    {
        uint64_t a = mk0, b = mk1;
#pragma unroll
        for (int k = 0; k < kStXr; ++k) {
            if ((uint32_t)k < nvec) {  // uniform
                const uint32_t sl = pop_slot(a, b);
                sv[k] = __builtin_amdgcn_raw_buffer_load_b128(
                    rh, tid < nw ? tid * 16 : kStOOB, __builtin_amdgcn_readfirstlane(sl * K * 2), 0);
            }
        }
    }
    // 2. prime the ring: a wave's first D items are row pairs p0 + wave,
    // + kStWaves, ... of the expert; every later one goes out through an LDS
    // counter to whichever wave refills a slot first (the SIMDs issue for
    // their older waves first, and a fixed deal left the younger waves
    // behind at the end). An item past the range loads through an empty
    // descriptor (no traffic, the same load count).
    const StLane<J> L = st_lane<J>(d.off_down, d, K, half * rowb, half * metab, half * 2);
    const rsrc_t r = make_rsrc(pool + (size_t)ex * d.blob, (uint32_t)d.blob);
    const rsrc_t rw0 = make_rsrc(pool + (size_t)ex * d.blob, 0u);
    constexpr int D = kPartD;
    static_assert(D == 3, "the loop body is written for three slots");
    StSlot<J> ring[D];
    uint32_t sk[D];  // the item (row pair - p0) each ring slot holds
    auto issue_k = [&](StSlot<J>& e, uint32_t k) __attribute__((always_inline)) {
        const bool ok = k < np;  // uniform
        const uint32_t pr = p0 + (ok ? k : 0u);
        st_issue<J>(e, ok ? r : rw0, L, 2 * pr * rowb, 2 * pr * metab, 2 * pr * 2);
    };
    // primed on every path (same load count: the staging waits only for its own loads)
#pragma unroll
    for (int q = 0; q < D; ++q) {
        sk[q] = wave + q * kStWaves;
        issue_k(ring[q], sk[q]);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (tid == 0) s_next = D * kStWaves;
    // 3. staging store: permuted pairs and chunk constants, chunks past K zero
#pragma unroll
    for (int k = 0; k < kStXr; ++k) {
        if ((uint32_t)k < nvec) {  // uniform
            float cs, cc;
            word_consts(sv[k], cs, cc);
            cs = quad_sum(cs);
            cc = quad_sum(cc);
            if (tid < nw) {
                const uint32_t ch = tid >> 2, jw = tid & 3;
                unsigned char* blk = act + (k * J + (ch >> 5)) * kABlk;
                *reinterpret_cast<u32x4*>(blk + jw * 512 + (ch & 31) * 16) = pair_perm(sv[k]);
                if (jw == 0)
                    *reinterpret_cast<float2*>(blk + 2048 + (ch & 31) * 8) = make_float2(cs, cc);
            }
        }
    }
    const uint32_t npad = 32 * J - nch;
    for (uint32_t i = tid; i < nvec * 5 * npad; i += blockDim.x) {
        const uint32_t v = i / (5 * npad), rem = i - v * 5 * npad, jw = rem / npad;
        const uint32_t ch = nch + (rem - jw * npad);
        unsigned char* blk = act + (v * J + (ch >> 5)) * kABlk;
        if (jw < 4) *reinterpret_cast<u32x4*>(blk + jw * 512 + (ch & 31) * 16) = u32x4{0, 0, 0, 0};
        else *reinterpret_cast<float2*>(blk + 2048 + (ch & 31) * 8) = make_float2(0.0f, 0.0f);
    }
    __syncthreads();

    if (wave >= np) return;  // no items; no later barrier

    // 4. stream
    const DequantConsts kc;
    // The draw: an LDS atomic by lane 0 alone, exec narrowed and restored
    // inside one asm block that also waits for the return (a one-lane atomic
    // written as a branch left the waitcnt pass waiting for every load at
    // the loop head; a return left in flight in a register past the asm could
    // be copied before it arrives); lane 0's value is made uniform outside it.
    const uint32_t next_a =
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)&s_next;
    auto draw = [&]() __attribute__((always_inline)) {
        uint32_t v;
        uint64_t saved;
        asm volatile(
            "s_mov_b64 %1, exec\n\t"
            "s_mov_b64 exec, 1\n\t"
            "ds_add_rtn_u32 %0, %2, %3\n\t"
            "s_mov_b64 exec, %1\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v), "=&s"(saved)
            : "v"(next_a), "v"(1u)
            : "memory");
        return __builtin_amdgcn_readfirstlane(v);
    };
    // One store per step by every lane: lane (h, j), j < nvec, writes slot j's
    // row 2 pr + h; the other lanes repeat the last slot's. The next ring wait
    // then does not also wait for it. A step draws the item its slot takes
    // next before its first use of the weights (far longer than an LDS atomic).
    auto step = [&](const StSlot<J>& e, uint32_t pr, uint32_t& nk) __attribute__((always_inline)) {
        __builtin_amdgcn_sched_barrier(0);
        nk = draw();
        __builtin_amdgcn_sched_barrier(0);
        StDq<J> q;
        st_dequant<J>(e, kc, q);
        const float b0 = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 0));
        const float b1 = bf2f((uint16_t)__builtin_amdgcn_readlane(e.bi, 32));
        uint64_t a = mk0, b = mk1;
        size_t oi = 0;
        float ov = 0.0f;
        for (uint32_t k = 0; k < nvec; ++k) {
            const uint32_t sl = pop_slot(a, b);
            const float2 hs = half_sums(st_dot<J>(q, act, k));
            const float wt = wgt[sl];
            if ((lane & 31) >= k) {
                oi = (size_t)sl * HID + 2 * pr + half;
                ov = wt * (half ? hs.y + b1 : hs.x + b0);
            }
        }
        ys[oi] = ov;
    };
    // a slot past the range stores once through an empty descriptor
    // (dropped) and refills out of range, so every path through the loop
    // issues the same stores and loads and each wait counts exactly the
    // other slots'
    const rsrc_t rnull = make_rsrc(ys, 0);
    auto slot = [&](int s, bool live) __attribute__((always_inline)) {
        uint32_t nk = np;
        if (live) step(ring[s], p0 + sk[s], nk);  // uniform
        else __builtin_amdgcn_raw_buffer_store_b32(0u, rnull, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        sk[s] = nk;
        issue_k(ring[s], nk);
        __builtin_amdgcn_sched_barrier(0);
    };
    // One exit, at the top (an exit after each slot let the compiler sink a
    // slot's refill loads past the next exit test). A slot past the range
    // means every later slot is, and so is the refilled slot 0.
    while (sk[0] < np) {  // uniform
        slot(0, true);
        slot(1, sk[1] < np);
        slot(2, sk[2] < np);
    }
}

// Y[t][m] = sum over k of ys[t * TK + k][m], in k order.
// ---------------------------------------------------------------------------
// 4. One-launch block (one token, KQ_MOE_PATH_ONE): router logits, top-k,
//    gate/up + SwiGLU and down + combine in a single launch of one 8-wave
//    workgroup per CU, with the three-launch block's results bit for bit.
//    The three-launch block pays two kernel boundaries and a plan read at
//    the start of each later launch. Measured at gpt-oss-120b shapes (12
//    layers, graph replays, same process): 21.87 us per block vs 21.94 us
//    for three launches -- the phase boundaries inside the launch (logit
//    exchange ~2.5 us, grid barrier ~1 us plus the down stream) cost about
//    what the kernel boundaries do, so the block stays on three launches by
//    default; this path saves two launches for callers that launch eagerly.
//    Streaming the down weights with gate/up (issued up front, or one item
//    per gate/up step) and deeper gate/up rings (3, 4: 22.19, 23.47 us) were
//    slower: the gate/up stream already runs at ~6.9 TB/s.
//    Here:
//    - each router wave stores its logit together with a tag (the call's
//      sequence number + 1) as one 8-byte device-coherent store, and wave 0
//      of every workgroup polls the tagged logits until all carry this
//      call's tag, then runs the top-k: the logits are their own barrier;
//    - each workgroup issues its share of the down rows into registers as
//      soon as its gate/up ring is primed, so the down weights stream with
//      gate/up;
//    - h goes to memory with device-coherent stores, one grid barrier
//      follows, and each wave loads the one h vector its down rows need
//      straight into registers (no LDS staging: down is one expert per wave,
//      two waves per expert at top-4).
//    x comes straight from memory into registers too.
//
//    Grid barrier: kSyncGroups 64-bit counters that only ever grow, one per
//    group of workgroups b % kSyncGroups, on separate lines: atomics on one
//    location are done in turn (measured per barrier at 256 workgroups: one
//    counter 3.7 us, 8 counters 2.0 us, 32 counters 1.0 us).
//    A workgroup arrives with one atomic add on its group's counter once its
//    device-coherent stores have completed; the value it gets back gives the
//    barrier round r (old / group size), and it waits until every counter
//    has reached (r + 1) x its group's size, polling all of them with one
//    load per lane. The round before a workgroup's own arrival is the call's
//    sequence number (its group cannot complete a round without it), which
//    gives the logit tag. The launch is sized so that all of its workgroups
//    are resident at once (one per CU, the occupancy query checked before the
//    first launch); every poll still gives up after kSpinTicks of the 100 MHz
//    real-time clock and sets the workspace's error word, so every wave
//    finishes.
// ---------------------------------------------------------------------------
constexpr size_t kWsErr = KQ_MOE_WS_ERR_OFFSET;  // head word (the plan is at 256)
constexpr uint64_t kSpinTicks = 10000000ull;     // 100 ms
// down items a wave holds in registers (2 at J = 4, within 256 VGPRs)
__host__ __device__ constexpr int one_dn(int J) { return J >= 4 ? 2 : 4; }
constexpr int kOneD = 2;  // gate/up ring depth

__device__ __forceinline__ uint32_t sync_gsize(uint32_t G, uint32_t g) {
    return G / kSyncGroups + (g < G % kSyncGroups ? 1u : 0u);
}
__device__ __forceinline__ void spin_fail(uint32_t* err) {
    if ((threadIdx.x & 63) == 0)
        __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival (thread 0, for the workgroup; the caller has made every thread's
// coherent stores complete and synchronised the workgroup) and wait, split
// so that work can be issued in between; the value the arrival returns goes
// to the wait.
__device__ __forceinline__ uint64_t grid_arrive(unsigned char* sync) {
    uint64_t old = 0;
    if (threadIdx.x == 0)
        old = __hip_atomic_fetch_add(
            reinterpret_cast<uint64_t*>(sync + (blockIdx.x % kSyncGroups) * kSyncStride), 1ull,
            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return old;
}
__device__ __forceinline__ void grid_wait(unsigned char* sync, uint32_t* err, uint64_t old) {
    if (threadIdx.x < 64) {  // wave 0 waits for the workgroup
        const uint32_t G = gridDim.x, lane = threadIdx.x, grp = blockIdx.x % kSyncGroups;
        const uint64_t old0 = ((uint64_t)__builtin_amdgcn_readlane((uint32_t)(old >> 32), 0) << 32) |
                              __builtin_amdgcn_readlane((uint32_t)old, 0);
        const uint64_t round = old0 / sync_gsize(G, grp);
        const bool mine = lane < kSyncGroups && sync_gsize(G, lane) > 0;
        const uint64_t target = (round + 1) * (mine ? sync_gsize(G, lane) : 0u);
        const uint64_t* cnt =
            reinterpret_cast<const uint64_t*>(sync + (mine ? lane : 0) * kSyncStride);
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (true) {
            bool done = true;
            if (mine)
                done = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target;
            if (__ballot(!done) == 0) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
                spin_fail(err);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// The J chunks of a K-element fp16 vector that lane c0 = lane % 32 uses
// (chunks c0 + 32j), loaded from memory into the register form st_xload
// gives (permuted pairs, chunk sum and offset constant; chunks past K zero).
// F32: the vector is fp32, rounded to fp16 here. AUX: cache policy of the
// loads. The chunk constants add the four words' constants as
// (w0 + w1) + (w2 + w3), the order of the staged form's quad sums.
template <int J, bool F32, int AUX>
__device__ __forceinline__ void st_xload_mem(StX<J>& x, const void* src, uint32_t K) {
    const uint32_t c0 = threadIdx.x & 31, nch = K >> 5;
    const rsrc_t r = make_rsrc(src, K * (F32 ? 4 : 2));
    u32x4 raw[J][4];
    f32x4 rf[F32 ? J : 1][F32 ? 8 : 1];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const uint32_t ch = c0 + 32 * j;
#pragma unroll
        for (int jw = 0; jw < 4; ++jw) {
            if constexpr (F32) {
                const uint32_t o = ch < nch ? ch * 128 + jw * 32 : kStOOB;
                rf[j][2 * jw] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, AUX));
                rf[j][2 * jw + 1] =
                    __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, o + 16, 0, AUX));
            } else {
                raw[j][jw] = __builtin_amdgcn_raw_buffer_load_b128(r, ch < nch ? ch * 64 + jw * 16 : kStOOB,
                                                                   0, AUX);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float sw[4], cw[4];
#pragma unroll
        for (int jw = 0; jw < 4; ++jw) {
            if constexpr (F32) {
                const f32x4 a = rf[j][2 * jw], b = rf[j][2 * jw + 1];
                raw[j][jw] = u32x4{(uint32_t)f2h(a.x) | ((uint32_t)f2h(a.y) << 16),
                                   (uint32_t)f2h(a.z) | ((uint32_t)f2h(a.w) << 16),
                                   (uint32_t)f2h(b.x) | ((uint32_t)f2h(b.y) << 16),
                                   (uint32_t)f2h(b.z) | ((uint32_t)f2h(b.w) << 16)};
            }
            word_consts(raw[j][jw], sw[jw], cw[jw]);
            x.p[j][jw] = pair_perm(raw[j][jw]);
        }
        x.k[j] = make_float2((sw[0] + sw[1]) + (sw[2] + sw[3]), (cw[0] + cw[1]) + (cw[2] + cw[3]));
    }
}

// The register form from the raw words st_xload_mem loads (fp16 vectors).
template <int J>
__device__ __forceinline__ void st_xregs(StX<J>& x, const u32x4 (&raw)[J][4]) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
        float sw[4], cw[4];
#pragma unroll
        for (int jw = 0; jw < 4; ++jw) {
            word_consts(raw[j][jw], sw[jw], cw[jw]);
            x.p[j][jw] = pair_perm(raw[j][jw]);
        }
        x.k[j] = make_float2((sw[0] + sw[1]) + (sw[2] + sw[3]), (cw[0] + cw[1]) + (cw[2] + cw[3]));
    }
}

// J: chunks per half-wave lane of both projections (hidden and inter of the
// same J); the router reads hidden in IT = 2J steps of 512 (IT * 512 >= hidden).
// rf32 / xf32: router weights / x in fp32 (uniform branches).
template <int J>
__global__ __launch_bounds__(64 * kStWaves) void moe_one_k(
    const uint8_t* __restrict__ pool, kq_moe_desc d, const void* __restrict__ R, int rf32,
    const void* __restrict__ X, int xf32, uint32_t* __restrict__ idx_out,
    float* __restrict__ wgt_out, uint16_t* __restrict__ xh, uint16_t* H, void* __restrict__ Y,
    int y_f32, unsigned char* sync, uint64_t* tagged, uint32_t* err, uint32_t pp) {
    extern __shared__ __align__(16) unsigned char act[];  // ys [top_k][2 pp]
    __shared__ Plan ps;
    __shared__ uint32_t s_idx[kMaxSlots];
    __shared__ float s_wgt[kMaxSlots];
    constexpr int IT = 2 * J;
    const uint32_t HID = d.hidden, IN = d.inter, TK = d.top_k, NE = d.n_experts, G = gridDim.x;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6), half = lane >> 5;

    // 1. router logits: expert e in wave e / G of workgroup e % G (spread over
    // the CUs), with the arithmetic of moe_router_k (the three-launch
    // block's logits); its loads go first, then the call's sequence number
    // (this workgroup's barrier counter), then x for gate/up
    const uint32_t e = wave * G + blockIdx.x;
    const uint32_t grp = blockIdx.x % kSyncGroups;
    const uint64_t* seq = reinterpret_cast<const uint64_t*>(sync + grp * kSyncStride);
    const bool router = e < NE;  // uniform
    u32x4 rr[IT][2], rx[IT][2];  // 8 router / x elements as loaded (fp32: two words)
    uint64_t seqv = 0;
    if (router) {
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            const uint32_t k = min((lane + 64 * i) * 8, HID - 8);
            if (rf32) {
                const u32x4* q = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(R) +
                                                                (size_t)e * HID + k);
                rr[i][0] = q[0];
                rr[i][1] = q[1];
            } else {
                rr[i][0] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(R) +
                                                           (size_t)e * HID + k);
            }
            if (xf32) {
                const u32x4* q = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(X) + k);
                rx[i][0] = q[0];
                rx[i][1] = q[1];
            } else {
                rx[i][0] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(X) + k);
            }
        }
    }
    if (router || wave == 0) seqv = __hip_atomic_load(seq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t tag = (uint32_t)(seqv / sync_gsize(G, grp)) + 1u;
    if (router) {
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < IT; ++i) {
            if ((lane + 64 * i) * 8 < HID) {
                float rv[8], xv[8];
                if (rf32) unpack8<true>(Raw8<true>{__builtin_bit_cast(f32x4, rr[i][0]),
                                                   __builtin_bit_cast(f32x4, rr[i][1])}, rv);
                else unpack8<false>(Raw8<false>{rr[i][0]}, rv);
                if (xf32) unpack8<true>(Raw8<true>{__builtin_bit_cast(f32x4, rx[i][0]),
                                                   __builtin_bit_cast(f32x4, rx[i][1])}, xv);
                else unpack8<false>(Raw8<false>{rx[i][0]}, xv);
#pragma unroll
                for (int q = 0; q < 8; ++q) acc = fmaf(rv[q], xv[q], acc);
            }
        }
        const float v = wave_sum(acc);
        const uint64_t tv = ((uint64_t)tag << 32) | __builtin_bit_cast(uint32_t, v);
        // one copy per XCD: the polls of each XCD's workgroups read their own
        if (lane < kTagCopies)
            __hip_atomic_store(tagged + lane * 256 + e, tv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (xf32 && xh)  // xh = half(X), spread over the grid
        for (uint32_t i = blockIdx.x * blockDim.x + tid; i < HID; i += G * blockDim.x)
            xh[i] = f2h(reinterpret_cast<const float*>(X)[i]);

    // 2. wave 0: wait for every logit of this call, top-k, the plan (one
    // token: the top-k experts are distinct, plan entry u is slot u)
    if (wave == 0) {
        const uint64_t* mine = tagged + (blockIdx.x % kTagCopies) * 256;
        float lv[4];
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        while (true) {
            uint64_t t[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)  // all four loads in flight at once
                t[q] = __hip_atomic_load(mine + min(lane + 64 * q, NE - 1), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
            bool done = true;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                lv[q] = __builtin_bit_cast(float, (uint32_t)t[q]);
                done = done && (uint32_t)(t[q] >> 32) == tag;
            }
            if (__ballot(!done) == 0) break;
            if (__builtin_amdgcn_s_memrealtime() - t0 > kSpinTicks) {
                spin_fail(err);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        topk_vals(lv, NE, TK, s_idx, s_wgt);
        __builtin_amdgcn_wave_barrier();
        if (lane < TK) {
            ps.expert[lane] = min(s_idx[lane], NE - 1);
            ps.mask[lane][0] = 1ull << lane;
            ps.mask[lane][1] = 0;
        }
        if (lane == 0) ps.n = TK;
        if (blockIdx.x == 0 && lane < TK) {
            idx_out[lane] = s_idx[lane];
            wgt_out[lane] = s_wgt[lane];
        }
    }
    __syncthreads();
    const uint32_t nexp = TK;
    // x (fp16) for gate/up, issued before any weight load (no later wait for
    // it waits for weights) and after the router's loads (not competing)
    const uint32_t c0 = lane & 31, nch = HID >> 5;
    u32x4 xraw[J][4];
    if (!xf32) {
        const rsrc_t r = make_rsrc(X, HID * 2);
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int jw = 0; jw < 4; ++jw) {
                const uint32_t ch = c0 + 32 * j;
                xraw[j][jw] =
                    __builtin_amdgcn_raw_buffer_load_b128(r, ch < nch ? ch * 64 + jw * 16 : kStOOB, 0, 0);
            }
    }

    // 3. gate/up items (u, row i), u-major, a contiguous range per workgroup,
    // every kStWaves-th item per wave (moe_gu_stream_k's order)
    const uint32_t N = nexp * IN;
    const uint32_t per = (N + G - 1) / G, k0 = blockIdx.x * per;
    const uint32_t cnt = k0 < N ? min(per, N - k0) : 0;
    const uint32_t nit = cnt > wave ? (cnt - wave + kStWaves - 1) / kStWaves : 0;
    const uint32_t rowb = HID >> 1, metab = (HID >> 6) * 2;
    const StLane<J> L = st_lane<J>(half ? d.off_up : d.off_gate, d, HID, 0, 0, 0);
    constexpr int D = kOneD;
    StSlot<J> ring[D];
    struct Cur {
        uint32_t u, i;
    };
    auto adv = [&](Cur& c) __attribute__((always_inline)) {
        c.i += kStWaves;
        while (c.i >= IN) {  // uniform
            c.i -= IN;
            ++c.u;
        }
    };
    Cur ci{(k0 + wave) / IN, (k0 + wave) % IN}, cc = ci, clast = ci;
    uint32_t nis = 0;
    auto issue = [&](StSlot<J>& sl) __attribute__((always_inline)) {
        if (nis < nit) clast = ci;  // padding re-reads the last item
        const uint32_t ex = __builtin_amdgcn_readfirstlane(ps.expert[min(clast.u, nexp - 1)]);
        const rsrc_t r = make_rsrc(pool + (size_t)ex * d.blob, (uint32_t)d.blob);
        const uint32_t i = __builtin_amdgcn_readfirstlane(clast.i);
        st_issue<J>(sl, r, L, i * rowb, i * metab, i * 2);
        adv(ci);
        ++nis;
    };
#pragma unroll
    for (int q = 0; q < D; ++q) {
        issue(ring[q]);
        __builtin_amdgcn_sched_barrier(0);
    }

    // 4. down items: wave q takes expert u = q % top_k and, among the W_u
    // waves of u, rank q / top_k: output row pairs p0 + rank + k W_u of this
    // workgroup's [p0, p0 + np), loaded into registers between the grid
    // barrier's arrival and its wait; items past the end load out of range
    // (no traffic)
    const uint32_t npairs = HID >> 1, p0 = blockIdx.x * pp;
    const uint32_t np = p0 < npairs ? min(pp, npairs - p0) : 0;
    const uint32_t du = wave % TK, drank = wave / TK;
    const uint32_t dW = kStWaves / TK + (du < kStWaves % TK ? 1u : 0u);
    const uint32_t rowd = IN >> 1, metad = (IN >> 6) * 2;
    const StLane<J> Ld = st_lane<J>(d.off_down, d, IN, half * rowd, half * metad, half * 2);
    const uint32_t dex = __builtin_amdgcn_readfirstlane(ps.expert[du]);
    constexpr int DN = one_dn(J);
    StSlot<J> dn[DN];
    auto issue_dn = [&](int k) __attribute__((always_inline)) {
        const uint32_t pi = drank + dW * k;
        const bool ok = pi < np;  // uniform
        const uint32_t p = p0 + (ok ? pi : 0);
        const rsrc_t r = make_rsrc(pool + (size_t)dex * d.blob, ok ? (uint32_t)d.blob : 0u);
        st_issue<J>(dn[k], r, Ld, 2 * p * rowd, 2 * p * metad, 2 * p * 2);
    };

    // x into registers
    StX<J> xr;
    if (xf32) st_xload_mem<J, true, 0>(xr, X, HID);
    else st_xregs<J>(xr, xraw);

    const DequantConsts kc;
    // every lane stores the step's h (the same value and address): a fixed
    // store count per step, device-coherent for the down phase's loads
    auto step = [&](const StSlot<J>& sl, uint32_t it, bool tail) __attribute__((always_inline)) {
        if (tail && it >= nit) return;  // padding (uniform)
        const float2 hs = half_sums(st_dotx_dq<J>(sl, kc, xr));
        const float bg = bf2f((uint16_t)__builtin_amdgcn_readlane(sl.bi, 0));
        const float bu = bf2f((uint16_t)__builtin_amdgcn_readlane(sl.bi, 32));
        const uint16_t hv = f2h(swiglu(hs.x + bg, hs.y + bu));
        __hip_atomic_store(H + (size_t)cc.u * IN + cc.i, hv, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        adv(cc);
    };
    const uint32_t nsteps = (nit + D - 1) / D * D;
    uint32_t it = 0;
    for (; it + D < nsteps; it += D) {
#pragma unroll
        for (int q = 0; q < D; ++q) {
            step(ring[q], it + q, false);
            issue(ring[q]);
        }
    }
#pragma unroll
    for (int q = 0; q < D; ++q) step(ring[q], it + q, true);
    // every wave's h stores complete, the workgroup arrives, then the down
    // loads go out (their fetch overlaps the wait). Issued any earlier --
    // before the gate/up tail, or by each wave right after its own h stores
    // with the arrival waiting for the stores alone -- they took bandwidth
    // from the slowest gate/up waves, which set the barrier: 21.7 -> 23.6 and
    // 22.9 us per block.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const uint64_t ticket = grid_arrive(sync);
#pragma unroll
    for (int k = 0; k < DN; ++k) issue_dn(k);

    __builtin_amdgcn_sched_barrier(0);
    grid_wait(sync, err, ticket);

    // 5. the wave's h vector (device-coherent loads) into registers, down
    // items, per-slot products to LDS, then the combine
    StX<J> hx;
    st_xload_mem<J, false, kCoh>(hx, H + (size_t)du * IN, IN);
    float* ys = reinterpret_cast<float*>(act);  // [TK][2 * pp]
    const float wt = s_wgt[du];
#pragma unroll
    for (int k = 0; k < DN; ++k) {
        const uint32_t pi = drank + dW * k;
        if (pi >= np) break;  // uniform
        const float2 hs = half_sums(st_dotx_dq<J>(dn[k], kc, hx));
        const float b0 = bf2f((uint16_t)__builtin_amdgcn_readlane(dn[k].bi, 0));
        const float b1 = bf2f((uint16_t)__builtin_amdgcn_readlane(dn[k].bi, 32));
        if (lane == 0) {
            ys[du * 2 * pp + 2 * pi] = wt * (hs.x + b0);
            ys[du * 2 * pp + 2 * pi + 1] = wt * (hs.y + b1);
        }
    }
    __syncthreads();
    // combine in slot order (moe-fused/src/kernels.metal:254-263)
    for (uint32_t i = tid; i < 2 * np; i += blockDim.x) {
        float acc = 0.0f;
        for (uint32_t q = 0; q < TK; ++q) acc += ys[q * 2 * pp + i];
        const uint32_t m = 2 * p0 + i;
        if (y_f32) reinterpret_cast<float*>(Y)[m] = acc;
        else reinterpret_cast<uint16_t*>(Y)[m] = f2h(acc);
    }
}

__global__ __launch_bounds__(256) void moe_combine_k(const float* __restrict__ ys, void* Y,
                                                     int y_f32, uint32_t batch, uint32_t TK,
                                                     uint32_t HID) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= batch * HID) return;
    const uint32_t t = i / HID, m = i - t * HID;
    float acc = 0.0f;
    for (uint32_t q = 0; q < TK; ++q) acc += ys[(size_t)(t * TK + q) * HID + m];
    if (y_f32) reinterpret_cast<float*>(Y)[i] = acc;
    else reinterpret_cast<uint16_t*>(Y)[i] = f2h(acc);
}

__global__ void fill_zero_k(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
        p[i] = 0u;
}

uint32_t chunks_j(uint32_t K) { return ((K >> 5) + 31) / 32; }

// Router outputs: the logits, and (with the tail) the completion counter and
// the plan; cnt and plan are unused without the tail.
struct RtOut {
    float* lg;
    uint32_t* cnt;
    Plan* plan;
    float* xsz = nullptr;  // zeroed by the router (the atomic block's sum(h)), nxs floats
    uint32_t nxs = 0;
};

template <int IT, bool TAIL>
hipError_t launch_router_it(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                            const kq_moe_desc& d, uint16_t* xh, RtOut o, uint32_t* idx,
                            float* wgt, hipStream_t s) {
    // with the tail: 4 waves (experts) per workgroup, so the last workgroup
    // has 4 waves for the per-token top-k; logits only: one wave per
    // workgroup, spreading the router's read over n_experts CUs
    constexpr int NW = TAIL ? 4 : 1;
    const dim3 grid((d.n_experts + NW - 1) / NW, (batch + 1) / 2);
    float* lg = o.lg;
    uint32_t* cnt = o.cnt;
    Plan* plan = o.plan;
#define KQ_RT(RF, XF)                                                                     \
    moe_router_k<RF, XF, IT, TAIL, NW><<<grid, 64 * NW, 0, s>>>(R, X, batch, d.n_experts, d.hidden, \
                                                         d.top_k, xh, lg, cnt, idx, wgt, plan,  \
                                                         o.xsz, o.nxs)
    if (r_f32 && x_f32) KQ_RT(true, true);
    else if (r_f32) KQ_RT(true, false);
    else if (x_f32) KQ_RT(false, true);
    else KQ_RT(false, false);
#undef KQ_RT
    return hipGetLastError();
}

template <bool TAIL>
hipError_t launch_router_o(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                           const kq_moe_desc& d, uint16_t* xh, RtOut o, uint32_t* idx, float* wgt,
                           hipStream_t s) {
    const uint32_t it = (d.hidden + 511) / 512;  // hidden <= 4096 (validated)
    if (it <= 2) return launch_router_it<2, TAIL>(R, r_f32, X, x_f32, batch, d, xh, o, idx, wgt, s);
    if (it <= 4) return launch_router_it<4, TAIL>(R, r_f32, X, x_f32, batch, d, xh, o, idx, wgt, s);
    if (it <= 6) return launch_router_it<6, TAIL>(R, r_f32, X, x_f32, batch, d, xh, o, idx, wgt, s);
    return launch_router_it<8, TAIL>(R, r_f32, X, x_f32, batch, d, xh, o, idx, wgt, s);
}

template <bool TAIL>
hipError_t launch_router_t(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                           const kq_moe_desc& d, uint16_t* xh, void* ws, uint32_t* idx, float* wgt,
                           hipStream_t s, bool zero_xsh = false) {
    const WsLayout L = ws_layout(d, batch);
    uint8_t* w = reinterpret_cast<uint8_t*>(ws);
    RtOut o{reinterpret_cast<float*>(w + L.lg), reinterpret_cast<uint32_t*>(w + L.cnt),
            reinterpret_cast<Plan*>(w + L.plan)};
    if (zero_xsh) {
        o.xsz = reinterpret_cast<float*>(w + L.xsh);
        o.nxs = batch * d.top_k * ((d.inter + 31) / 32);
    }
    return launch_router_o<TAIL>(R, r_f32, X, x_f32, batch, d, xh, o, idx, wgt, s);
}

// Router with its tail: logits, then (last workgroup) top-k, idx/wgt and plan.
hipError_t launch_router(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                         const kq_moe_desc& d, uint16_t* xh, void* ws, uint32_t* idx, float* wgt,
                         hipStream_t s) {
    return launch_router_t<true>(R, r_f32, X, x_f32, batch, d, xh, ws, idx, wgt, s);
}

template <int J, bool FP>
hipError_t go_gu(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx, const Plan* plan,
                 const uint16_t* xh, uint16_t* H, uint32_t batch, hipStream_t s) {
    const uint32_t nslots = batch * d.top_k;
    const dim3 grid((d.inter + kGuRows - 1) / kGuRows, nslots < d.n_experts ? nslots : d.n_experts);
    moe_gate_up_k<J, FP><<<grid, kGuThreads, 0, s>>>(pool, d, idx, plan, xh, H, batch);
    return hipGetLastError();
}

constexpr size_t kStStatic = sizeof(Plan) + 2 * kMaxSlots * 4 + 64;  // static LDS, rounded up
constexpr size_t kLdsMax = 160 * 1024;

template <typename Kern>
hipError_t st_lds(Kern kern, size_t lds) {
    if (lds <= 64 * 1024) return hipSuccess;
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

// The streaming kernels take activation vectors staged in one pass, with
// room in LDS, and an expert blob addressable with 32-bit offsets.
bool st_ok(const kq_moe_desc& d, uint32_t nvec, uint32_t K, size_t extra) {
    return d.blob < (1ull << 31) && (size_t)nvec * (K >> 3) <= (size_t)kStXr * 64 * kStWaves &&
           st_act_bytes(nvec, K) + extra + kStStatic <= kLdsMax;
}

// The atomic block's per-workgroup sums of h in the streaming gate/up's LDS:
// slots x the chunks a workgroup's items can span -- per = its share of at
// most batch x top_k experts' rows spans at most per / 32 + 2 chunks of one
// expert plus one per expert boundary (at most per / inter + 1), one more for
// rounding.
size_t gu_sums_lds(const kq_moe_desc& d, uint32_t batch) {
    const uint32_t nsl = batch * d.top_k, G = cu_count();
    const uint32_t per = (nsl * d.inter + G - 1) / G;
    return (size_t)nsl * (per / 32 + 4 + per / d.inter) * 4;
}

// Top-k in the gate/up launch (SRC 2): the logits, and where idx / wgt /
// plan go.
struct GuTopk {
    const float* lg;
    uint32_t* idx;
    float* wgt;
    Plan* plan;
};

template <int J, int SRC, bool AT = false>
hipError_t go_gu_st(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                    const Plan* plan, const uint16_t* xh, uint16_t* H, uint32_t batch,
                    GuTopk tk, hipStream_t s, float* xsh = nullptr) {
    const uint32_t G = cu_count();
    const size_t lds = st_act_bytes(batch, d.hidden) + (AT ? gu_sums_lds(d, batch) : 0);
    auto run = [&](auto kern) {
        const hipError_t e = st_lds(kern, lds);
        if (e != hipSuccess) return e;
        kern<<<G, 64 * kStWaves, lds, s>>>(pool, d, idx, plan, xh, H, batch, tk.lg,
                                            tk.idx, tk.wgt, tk.plan, xsh);
        return hipGetLastError();
    };
    return batch == 1 ? run(moe_gu_stream_k<J, SRC, true, AT>) : run(moe_gu_stream_k<J, SRC, false, AT>);
}

template <int J, bool FP, bool AT = false>
hipError_t go_dn_st(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                    const float* wgt, const Plan* plan, const uint16_t* H, void* Y, bool y_f32,
                    uint32_t batch, uint32_t pp, hipStream_t s, const float* xsh = nullptr) {
    auto kern = moe_dn_stream_k<J, FP, AT>;
    const uint32_t nslots = batch * d.top_k, npairs = d.hidden / 2;
    const size_t lds = st_act_bytes(nslots, d.inter) + (size_t)nslots * 2 * pp * 4;
    const hipError_t e = st_lds(kern, lds);
    if (e != hipSuccess) return e;
    kern<<<(npairs + pp - 1) / pp, 64 * kStWaves, lds, s>>>(pool, d, idx, wgt, plan, H, Y,
                                                             y_f32 ? 1 : 0, batch, pp, xsh);
    return hipGetLastError();
}

// Streaming gate/up: measured (gpt-oss shapes) 12.0 us vs per-tile 13.9 us
// at one token; at 8 tokens the per-tile kernel wins (69.5 vs 78.5 us).
bool gu_streams(const kq_moe_desc& d, uint32_t batch) {
    // batch * top_k <= kPlanSlots: the in-kernel top-k's plan limit
    return batch <= 2 && st_ok(d, batch, d.hidden, 0);
}

// The block's gate/up streams at one token only. Whole block, gpt-oss-120b
// shapes: at one token streaming 21.8 us, expert-partitioned 22.3 us; at two
// tokens streaming 34.3 us, expert-partitioned 31.9 us.
bool block_gu_streams(const kq_moe_desc& d, uint32_t batch) {
    return batch == 1 && gu_streams(d, batch);
}

template <int SRC, bool AT = false>
hipError_t launch_gu_st(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                        const Plan* plan, const uint16_t* xh, uint16_t* H, uint32_t batch,
                        GuTopk tk, hipStream_t s, float* xsh = nullptr) {
    switch (chunks_j(d.hidden)) {
        case 1: return go_gu_st<1, SRC, AT>(pool, d, idx, plan, xh, H, batch, tk, s, xsh);
        case 2: return go_gu_st<2, SRC, AT>(pool, d, idx, plan, xh, H, batch, tk, s, xsh);
        case 3: return go_gu_st<3, SRC, AT>(pool, d, idx, plan, xh, H, batch, tk, s, xsh);
        case 4: return go_gu_st<4, SRC, AT>(pool, d, idx, plan, xh, H, batch, tk, s, xsh);
        default: return hipErrorInvalidValue;
    }
}

// One round: one workgroup per CU (the partitioned kernels run one 8-wave
// workgroup per CU at their register use), and at least one per plan entry.
uint32_t part_grid(const kq_moe_desc& d, uint32_t batch) {
    const uint32_t nslots = batch * d.top_k;
    const uint32_t nu = nslots < d.n_experts ? nslots : d.n_experts;  // plan entries at most
    return cu_count() > nu ? cu_count() : nu;
}

template <int J>
hipError_t go_gu_part(const uint8_t* pool, const kq_moe_desc& d, const uint16_t* xh, uint16_t* H,
                      uint32_t batch, GuTopk tk, hipStream_t s) {
    auto kern = moe_gu_part_k<J>;
    const size_t lds = st_act_bytes(batch, d.hidden);  // every token's x
    const hipError_t e = st_lds(kern, lds);
    if (e != hipSuccess) return e;
    kern<<<part_grid(d, batch), 64 * kStWaves, lds, s>>>(pool, d, xh, batch, H, tk.lg, tk.idx,
                                                          tk.wgt, tk.plan);
    return hipGetLastError();
}

hipError_t launch_gu_part(const uint8_t* pool, const kq_moe_desc& d, const uint16_t* xh,
                          uint16_t* H, uint32_t batch, GuTopk tk, hipStream_t s) {
    switch (chunks_j(d.hidden)) {
        case 1: return go_gu_part<1>(pool, d, xh, H, batch, tk, s);
        case 2: return go_gu_part<2>(pool, d, xh, H, batch, tk, s);
        case 3: return go_gu_part<3>(pool, d, xh, H, batch, tk, s);
        case 4: return go_gu_part<4>(pool, d, xh, H, batch, tk, s);
        default: return hipErrorInvalidValue;
    }
}

// The expert-partitioned gate/up: every token's x staged in one pass (at
// most kStXr words per thread) and in LDS next to the plan.
bool gu_part_ok(const kq_moe_desc& d, uint32_t batch) {
    return batch <= (uint32_t)kStXr && (d.hidden >> 3) <= 64u * kStWaves &&
           d.blob < (1ull << 31) && st_act_bytes(batch, d.hidden) + kStStatic <= kLdsMax;
}

template <bool FP>
hipError_t launch_gu(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                     const Plan* plan, const uint16_t* xh, uint16_t* H, uint32_t batch,
                     hipStream_t s) {
    if (gu_streams(d, batch))
        return launch_gu_st<FP ? 1 : 0>(pool, d, idx, plan, xh, H, batch, GuTopk{}, s);
    switch (chunks_j(d.hidden)) {
        case 1: return go_gu<1, FP>(pool, d, idx, plan, xh, H, batch, s);
        case 2: return go_gu<2, FP>(pool, d, idx, plan, xh, H, batch, s);
        case 3: return go_gu<3, FP>(pool, d, idx, plan, xh, H, batch, s);
        case 4: return go_gu<4, FP>(pool, d, idx, plan, xh, H, batch, s);
        default: return hipErrorInvalidValue;
    }
}

// One round of cost-weighted row chunks (part_assign), then the combine.
template <int J>
hipError_t go_dn_part(const uint8_t* pool, const kq_moe_desc& d, const float* wgt,
                      const Plan* plan, const uint16_t* H, void* Y, bool y_f32, uint32_t batch,
                      float* ys, hipStream_t s) {
    auto kern = moe_dn_part_k<J>;
    const uint32_t nslots = batch * d.top_k;
    const size_t lds = st_act_bytes(batch, d.inter);  // at most one slot per token per expert
    hipError_t e = st_lds(kern, lds);
    if (e != hipSuccess) return e;
    kern<<<part_grid(d, batch), 64 * kStWaves, lds, s>>>(pool, d, wgt, plan, H, nslots, ys);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const uint32_t n = batch * d.hidden;
    moe_combine_k<<<(n + 255) / 256, 256, 0, s>>>(ys, Y, y_f32 ? 1 : 0, batch, d.top_k, d.hidden);
    return hipGetLastError();
}

// The expert-partitioned down: up to kStXr tokens (the h vectors a thread
// stages), inter <= one word per thread, the h blocks in LDS.
bool dn_part_ok(const kq_moe_desc& d, uint32_t batch) {
    return batch <= (uint32_t)kStXr && (d.inter >> 3) <= 64u * kStWaves &&
           d.blob < (1ull << 31) && st_act_bytes(batch, d.inter) + 1024 <= kLdsMax;
}

// ys: workspace for the per-slot products (nullptr: not available).
template <bool FP>
hipError_t launch_dn(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                     const float* wgt, const Plan* plan, const uint16_t* H, void* Y, bool y_f32,
                     uint32_t batch, hipStream_t s, float* ys = nullptr) {
    const uint32_t nslots = batch * d.top_k, npairs = d.hidden / 2;
    const uint32_t pp = (npairs + cu_count() - 1) / cu_count();
    if constexpr (FP) {
        if (ys && !st_ok(d, nslots, d.inter, (size_t)nslots * 2 * pp * 4) && dn_part_ok(d, batch)) {
            switch (chunks_j(d.inter)) {
                case 1: return go_dn_part<1>(pool, d, wgt, plan, H, Y, y_f32, batch, ys, s);
                case 2: return go_dn_part<2>(pool, d, wgt, plan, H, Y, y_f32, batch, ys, s);
                case 3: return go_dn_part<3>(pool, d, wgt, plan, H, Y, y_f32, batch, ys, s);
                case 4: return go_dn_part<4>(pool, d, wgt, plan, H, Y, y_f32, batch, ys, s);
                default: return hipErrorInvalidValue;
            }
        }
    }
    if (st_ok(d, nslots, d.inter, (size_t)nslots * 2 * pp * 4)) {
        switch (chunks_j(d.inter)) {
            case 1: return go_dn_st<1, FP>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s);
            case 2: return go_dn_st<2, FP>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s);
            case 3: return go_dn_st<3, FP>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s);
            case 4: return go_dn_st<4, FP>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s);
            default: return hipErrorInvalidValue;
        }
    }
    const dim3 grid((d.hidden + kDnRows - 1) / kDnRows);
    const int yf = y_f32 ? 1 : 0;
#define KQ_DN(JJ) \
    moe_down_k<JJ, FP><<<grid, kDnThreads, 0, s>>>(pool, d, idx, wgt, plan, H, Y, yf, batch)
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

// One-launch block limits: one token; hidden and inter of one chunk count
// per lane; every wave's down items within its registers; the router's
// experts within the grid's waves.
uint32_t one_pp(const kq_moe_desc& d) {
    const uint32_t G = cu_count();
    return (d.hidden / 2 + G - 1) / G;
}
size_t one_lds(const kq_moe_desc& d) { return (size_t)d.top_k * 2 * one_pp(d) * 4; }
bool one_fits(const kq_moe_desc& d, uint32_t batch) {
    const uint32_t J = chunks_j(d.hidden);
    if (batch != 1 || J < 1 || J > 4 || chunks_j(d.inter) != J || cu_count() >= 0x10000u)
        return false;
    const uint32_t wmin = (uint32_t)kStWaves / d.top_k;  // waves per expert (top_k <= 8)
    return wmin >= 1 && (one_pp(d) + wmin - 1) / wmin <= (uint32_t)one_dn((int)J) &&
           d.n_experts <= cu_count() * (uint32_t)kStWaves && d.blob < (1ull << 31) &&
           one_lds(d) + kStStatic <= kLdsMax;
}
const void* one_kern(uint32_t J) {
    switch (J) {
        case 1: return reinterpret_cast<const void*>(moe_one_k<1>);
        case 2: return reinterpret_cast<const void*>(moe_one_k<2>);
        case 3: return reinterpret_cast<const void*>(moe_one_k<3>);
        case 4: return reinterpret_cast<const void*>(moe_one_k<4>);
        default: return nullptr;
    }
}

// Every workgroup of the launch (one per CU) resident at once: the occupancy
// query, once per (device, kernel, LDS size).
struct OneRes {
    int dev;
    const void* kern;
    size_t lds;
    bool ok;
};
std::mutex g_one_mu;
OneRes g_one_res[64];
int g_one_n = 0;
bool one_resident(const void* kern, size_t lds) {
    int dev = 0;
    if (kern == nullptr || hipGetDevice(&dev) != hipSuccess) return false;
    std::lock_guard<std::mutex> lk(g_one_mu);
    for (int i = 0; i < g_one_n; ++i)
        if (g_one_res[i].dev == dev && g_one_res[i].kern == kern && g_one_res[i].lds == lds)
            return g_one_res[i].ok;
    int nb = 0;
    const bool ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kern, 64 * kStWaves, lds) ==
                        hipSuccess &&
                    nb >= 1;
    if (g_one_n < 64) g_one_res[g_one_n++] = OneRes{dev, kern, lds, ok};
    return ok;
}

template <int J>
hipError_t go_one(const uint8_t* pool, const kq_moe_desc& d, const void* R, bool rf,
                  const void* X, bool xf, uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H,
                  void* Y, bool y_f32, uint8_t* w, const WsLayout& L, hipStream_t s) {
    auto kern = moe_one_k<J>;
    const size_t lds = one_lds(d);
    const hipError_t e = st_lds(kern, lds);
    if (e != hipSuccess) return e;
    kern<<<cu_count(), 64 * kStWaves, lds, s>>>(
        pool, d, R, rf ? 1 : 0, X, xf ? 1 : 0, idx, wgt, xh, H, Y, y_f32 ? 1 : 0, w + L.sync,
        reinterpret_cast<uint64_t*>(w + L.tag), reinterpret_cast<uint32_t*>(w + kWsErr), one_pp(d));
    return hipGetLastError();
}
hipError_t launch_one(const uint8_t* pool, const kq_moe_desc& d, const void* R, bool rf,
                      const void* X, bool xf, uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H,
                      void* Y, bool y_f32, uint8_t* w, const WsLayout& L, hipStream_t s) {
    switch (chunks_j(d.hidden)) {
        case 1: return go_one<1>(pool, d, R, rf, X, xf, idx, wgt, xh, H, Y, y_f32, w, L, s);
        case 2: return go_one<2>(pool, d, R, rf, X, xf, idx, wgt, xh, H, Y, y_f32, w, L, s);
        case 3: return go_one<3>(pool, d, R, rf, X, xf, idx, wgt, xh, H, Y, y_f32, w, L, s);
        case 4: return go_one<4>(pool, d, R, rf, X, xf, idx, wgt, xh, H, Y, y_f32, w, L, s);
        default: return hipErrorInvalidValue;
    }
}

// Per-device address of `scratch`, looked up once per device (with that
// device current) at the first kq_moe_block_noalloc call on it. Nothing is
// enqueued for the set-up: the array has static storage and no initialiser,
// so the loader gives every GPU's copy zeros, which is what the block needs
// (its only state carried from call to call, the router tail's completion
// counter, returns to zero at the end of every call). A first call made
// under stream capture therefore records only the block's own kernels.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

hipError_t scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch[dev] == nullptr) {
        void* p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return hipSuccess;
}

}  // namespace

// The atomic sum(h) block: the streaming gate/up (1-2 tokens) and the
// streaming down, whose staging takes the sums.
bool moe_atomic_supported(const kq_moe_desc& d, uint32_t batch) {
    if (!gu_streams(d, batch) || chunks_j(d.inter) < 1 || chunks_j(d.inter) > 4) return false;
    if (!st_ok(d, batch, d.hidden, gu_sums_lds(d, batch))) return false;
    const uint32_t nslots = batch * d.top_k, pp = (d.hidden / 2 + cu_count() - 1) / cu_count();
    return st_ok(d, nslots, d.inter, (size_t)nslots * 2 * pp * 4);
}

bool moe_one_supported(const kq_moe_desc& d, uint32_t batch) {
    return one_fits(d, batch) && one_resident(one_kern(chunks_j(d.hidden)), one_lds(d));
}

hipError_t launch_moe_block_noalloc(const uint8_t* pool, const kq_moe_desc& d, const void* R,
                                    bool r_f32, const void* X, bool x_f32, uint32_t batch,
                                    uint32_t* idx, float* wgt, uint16_t* xh, uint16_t* H, void* Y,
                                    bool y_f32, hipStream_t s) {
    void* ws = nullptr;
    const hipError_t e = scratch_ptr(&ws);
    if (e != hipSuccess) return e;
    return launch_moe_block(pool, d, R, r_f32, X, x_f32, batch, idx, wgt, xh, H, Y, y_f32, ws, s,
                            KQ_MOE_PATH_AUTO);
}

hipError_t launch_moe_logits(const void* R, bool r_f32, const void* X, bool x_f32, uint32_t batch,
                             const kq_moe_desc& d, uint16_t* xh, float* lg, hipStream_t s) {
    return launch_router_o<false>(R, r_f32, X, x_f32, batch, d, xh, RtOut{lg, nullptr, nullptr},
                                  nullptr, nullptr, s);
}

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
    return launch_router(R, r_f32, X, x_f32, batch, d, xh, ws, idx, wgt, s);
}

hipError_t launch_moe_gate_up(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                              const uint16_t* xh, uint16_t* H, uint32_t batch, hipStream_t s) {
    return launch_gu<false>(pool, d, idx, nullptr, xh, H, batch, s);
}

hipError_t launch_moe_down(const uint8_t* pool, const kq_moe_desc& d, const uint32_t* idx,
                           const float* wgt, const uint16_t* H, void* Y, bool y_f32,
                           uint32_t batch, hipStream_t s) {
    return launch_dn<false>(pool, d, idx, wgt, nullptr, H, Y, y_f32, batch, s);
}

// The block: three launches (KQ_MOE_PATH_ONE: the one-launch kernel). With
// the streaming gate/up (one token; the atomic form, 1-2 tokens) the
// router's top-k tail moves into the gate/up launch: every gate/up workgroup
// selects from the logits (cheap, L2-resident) instead of the router's last
// workgroup doing it after a device-scope hand-off (measured 8.1 -> 3.3 us
// for the router at one token).
hipError_t launch_moe_block(const uint8_t* pool, const kq_moe_desc& d, const void* R, bool r_f32,
                            const void* X, bool x_f32, uint32_t batch, uint32_t* idx, float* wgt,
                            uint16_t* xh, uint16_t* H, void* Y, bool y_f32, void* ws,
                            hipStream_t s, int path) {
    const WsLayout L = ws_layout(d, batch);
    uint8_t* w = reinterpret_cast<uint8_t*>(ws);
    if (path == KQ_MOE_PATH_ONE)
        return launch_one(pool, d, R, r_f32, X, x_f32, idx, wgt, xh, H, Y, y_f32, w, L, s);
    Plan* plan = reinterpret_cast<Plan*>(w + L.plan);
    const uint16_t* xin = x_f32 ? xh : reinterpret_cast<const uint16_t*>(X);
    hipError_t e;
    if (path == KQ_MOE_PATH_ATOMIC) {  // callers check moe_atomic_supported
        float* xsh = reinterpret_cast<float*>(w + L.xsh);
        e = launch_router_t<false>(R, r_f32, X, x_f32, batch, d, xh, ws, idx, wgt, s, true);
        if (e != hipSuccess) return e;
        const GuTopk tk{reinterpret_cast<const float*>(w + L.lg), idx, wgt, plan};
        e = launch_gu_st<2, true>(pool, d, idx, plan, xin, H, batch, tk, s, xsh);
        if (e != hipSuccess) return e;
        const uint32_t pp = (d.hidden / 2 + cu_count() - 1) / cu_count();
        switch (chunks_j(d.inter)) {
            case 1: return go_dn_st<1, true, true>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s, xsh);
            case 2: return go_dn_st<2, true, true>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s, xsh);
            case 3: return go_dn_st<3, true, true>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s, xsh);
            case 4: return go_dn_st<4, true, true>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, pp, s, xsh);
            default: return hipErrorInvalidValue;
        }
    }
    if (block_gu_streams(d, batch)) {
        e = launch_router_t<false>(R, r_f32, X, x_f32, batch, d, xh, ws, idx, wgt, s);
        if (e != hipSuccess) return e;
        const GuTopk tk{reinterpret_cast<const float*>(w + L.lg), idx, wgt, plan};
        e = launch_gu_st<2>(pool, d, idx, plan, xin, H, batch, tk, s);
    } else if (gu_part_ok(d, batch)) {
        // logits only; every partitioned gate/up workgroup runs the top-k
        // and builds the plan, workgroup 0 publishes it (measured at 8
        // tokens: the router with its device-wide top-k tail took 11.5 us)
        e = launch_router_t<false>(R, r_f32, X, x_f32, batch, d, xh, ws, idx, wgt, s);
        if (e != hipSuccess) return e;
        const GuTopk tk{reinterpret_cast<const float*>(w + L.lg), idx, wgt, plan};
        e = launch_gu_part(pool, d, xin, H, batch, tk, s);
    } else {
        e = launch_router(R, r_f32, X, x_f32, batch, d, xh, ws, idx, wgt, s);
        if (e != hipSuccess) return e;
        e = launch_gu<true>(pool, d, idx, plan, xin, H, batch, s);
    }
    if (e != hipSuccess) return e;
    return launch_dn<true>(pool, d, idx, wgt, plan, H, Y, y_f32, batch, s,
                           reinterpret_cast<float*>(w + L.ys));
}

}  // namespace kq
