// kq_moe_device.h -- device helpers shared by the three-launch MoE block
// (kq_moe.hip) and its one-op-per-launch form (kq_moe_unfused.hip): the
// wave top-k selection of the router and the SwiGLU activation.
#pragma once
#include "kq_device.h"

namespace kq {

// Candidate logit as the selection sees it: NaN, -inf and past-the-end
// experts are never selectable (-inf); -0 counts as +0, so equal logits tie.
__device__ __forceinline__ float cand(float v, bool valid) {
    return valid && v > -INFINITY ? v + 0.0f : -INFINITY;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_fmax(float x) {
    const int xi = __builtin_bit_cast(int, x);
    const int o = __builtin_amdgcn_update_dpp(xi, xi, CTRL, ROW_MASK, 0xF, false);
    return fmaxf(x, __builtin_bit_cast(float, o));
}

// Largest value of the wave, uniform (DPP butterfly, then lane 63).
__device__ __forceinline__ float wave_max_f32(float x) {
    x = dpp_fmax<0xB1, 0xF>(x);   // xor 1
    x = dpp_fmax<0x4E, 0xF>(x);   // xor 2
    x = dpp_fmax<0x124, 0xF>(x);  // row_ror 4
    x = dpp_fmax<0x128, 0xF>(x);  // row_ror 8
    x = dpp_fmax<0x142, 0xA>(x);  // row_bcast 15
    x = dpp_fmax<0x143, 0xC>(x);  // row_bcast 31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}

// Top-k by repeated argmax over one wave's candidates, v[q] = the logit of
// expert lane + 64 q (as cand() maps it), as the reference does it
// (moe-fused/src/kernels.metal:149-156): pass j takes the largest remaining
// value -- the lowest index among equal values, as a strictly-greater
// ascending scan does -- and removes it; a pass with nothing selectable
// yields index 0 and -inf. Each pass is one float max reduction and a ballot
// per candidate column (lowest column first, then lowest lane). pick[] and
// chosen[] are uniform.
template <int KMAX>
__device__ __forceinline__ void topk_select(float (&v)[4], uint32_t TK, uint32_t (&pick)[KMAX],
                                            float (&chosen)[KMAX]) {
    const uint32_t lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        pick[j] = 0;
        chosen[j] = -INFINITY;
        if ((uint32_t)j >= TK) continue;  // uniform
        const float mx = wave_max_f32(fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3])));
        if (mx == -INFINITY) continue;  // nothing selectable (uniform)
        uint32_t bi = 0;
        bool found = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint64_t b = __ballot(v[q] == mx);
            if (!found && b != 0) {
                bi = 64 * q + (uint32_t)__builtin_ctzll(b);
                found = true;
            }
        }
        pick[j] = bi;
        chosen[j] = mx;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (lane + 64 * q == bi) v[q] = -INFINITY;
    }
}

// SwiGLU of the reference (moe-fused/src/kernels.metal:177-215): the gate
// clamped above at 7, the up value to [-7, 7], alpha 1.702, (up + 1).
__device__ __forceinline__ float swiglu(float g, float u) {
    const float gg = fminf(g, 7.0f), uu = fminf(fmaxf(u, -7.0f), 7.0f);
    return gg * __frcp_rn(1.0f + __expf(-1.702f * gg)) * (uu + 1.0f);
}

}  // namespace kq
