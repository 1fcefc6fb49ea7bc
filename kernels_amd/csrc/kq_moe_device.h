// kq_moe_device.h -- device helpers shared by the three-launch MoE block
// (kq_moe.hip) and its one-op-per-launch form (kq_moe_unfused.hip): the
// wave argmax of the router top-k and the SwiGLU activation.
#pragma once
#include "kq_device.h"

namespace kq {

// Order key of a candidate: larger key = better. Selectable logits (not NaN,
// not -inf) map to an order-preserving unsigned code in the high word (always
// > 0; -0 counts as +0 so equal logits tie), unselectable ones to 0; the low
// word is ~index, so among equal high words the lowest index is the largest.
__device__ __forceinline__ uint64_t cand_key(float v, uint32_t e) {
    uint32_t hi = 0;
    if (v > -INFINITY) {
        const uint32_t b = __builtin_bit_cast(uint32_t, v + 0.0f);
        hi = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return ((uint64_t)hi << 32) | (uint32_t)~e;
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_max_u64(uint64_t k) {
    const int lo = (int)(uint32_t)k, hi = (int)(uint32_t)(k >> 32);
    const uint32_t olo = (uint32_t)__builtin_amdgcn_update_dpp(lo, lo, CTRL, ROW_MASK, 0xF, false);
    const uint32_t ohi = (uint32_t)__builtin_amdgcn_update_dpp(hi, hi, CTRL, ROW_MASK, 0xF, false);
    const uint64_t o = ((uint64_t)ohi << 32) | olo;
    return o > k ? o : k;
}

// Largest key of the wave, uniform (DPP butterfly, then lane 63).
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    k = dpp_max_u64<0xB1, 0xF>(k);   // xor 1
    k = dpp_max_u64<0x4E, 0xF>(k);   // xor 2
    k = dpp_max_u64<0x124, 0xF>(k);  // row_ror 4
    k = dpp_max_u64<0x128, 0xF>(k);  // row_ror 8
    k = dpp_max_u64<0x142, 0xA>(k);  // row_bcast 15
    k = dpp_max_u64<0x143, 0xC>(k);  // row_bcast 31
    const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)k, 63);
    const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

// SwiGLU of the reference (moe-fused/src/kernels.metal:177-215): the gate
// clamped above at 7, the up value to [-7, 7], alpha 1.702, (up + 1).
__device__ __forceinline__ float swiglu(float g, float u) {
    const float gg = fminf(g, 7.0f), uu = fminf(fmaxf(u, -7.0f), 7.0f);
    return gg * __frcp_rn(1.0f + __expf(-1.702f * gg)) * (uu + 1.0f);
}

}  // namespace kq
