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

// Order-preserving key of a candidate (as cand() maps it): 0 for -inf (never
// selectable); any other value keeps its bits with the sign bit flipped if
// it is positive, or every bit flipped if it is negative. Unsigned order of
// the keys is then the floats' order, and equal keys are equal floats (+0 is
// the only zero a candidate can be). Bits compare exactly, denormals included.
__device__ __forceinline__ uint32_t cand_key(float v) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    return v == -INFINITY ? 0u : b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {  // the candidate of key k != 0
    return __builtin_bit_cast(float, (k & 0x80000000u) ? k ^ 0x80000000u : ~k);
}

// Sum with a DPP-moved copy. Every lane's source lies in its own row (quad
// permutes, half-row mirror), so the move needs no old value and can fold
// into the add.
template <int CTRL>
__device__ __forceinline__ float dpp_fadd(float x) {
    const int o = __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true);
    return x + __builtin_bit_cast(float, o);
}

// Descending lists of L candidate keys per lane, merged across lanes. A
// merge of two descending lists a and b keeps c_i = max(a_i, b_{L-1-i}):
// the L largest of both, in a bitonic order that the half-cleaner network
// below sorts (compare-exchange of i and i + h for h = L/2, ..., 1).
template <int L>
__device__ __forceinline__ void bitonic_sort_desc(uint32_t (&c)[L]) {
#pragma unroll
    for (int h = L / 2; h >= 1; h >>= 1)
#pragma unroll
        for (int i = 0; i < L; ++i)
            if ((i & h) == 0) {
                const uint32_t x = c[i], y = c[i + h];
                c[i] = max(x, y);
                c[i + h] = min(x, y);
            }
}
// Merge with the list of the lane a DPP pattern within the row names (every
// source lane valid, so the move folds into the max).
template <int L, int CTRL>
__device__ __forceinline__ void list_merge_dpp(uint32_t (&a)[L]) {
    uint32_t c[L];
#pragma unroll
    for (int i = 0; i < L; ++i)
        c[i] = max(a[i], (uint32_t)__builtin_amdgcn_mov_dpp((int)a[L - 1 - i], CTRL, 0xF, 0xF, true));
    bitonic_sort_desc(c);
#pragma unroll
    for (int i = 0; i < L; ++i) a[i] = c[i];
}
// Merge across rows: v_permlane16_swap of a register with itself gives every
// lane the lists of rows 0 / 2 and of rows 1 / 3 of its row pair, and
// v_permlane32_swap the lists of the lower and the upper half; each lane
// merges the two (the same result in both partners).
template <int L, bool HALVES>
__device__ __forceinline__ void list_merge_swap(uint32_t (&a)[L]) {
    uint32_t lo[L], hi[L];
#pragma unroll
    for (int i = 0; i < L; ++i) {
        if constexpr (HALVES) {
            const auto r = __builtin_amdgcn_permlane32_swap(a[i], a[i], false, false);
            lo[i] = r[0];
            hi[i] = r[1];
        } else {
            const auto r = __builtin_amdgcn_permlane16_swap(a[i], a[i], false, false);
            lo[i] = r[0];
            hi[i] = r[1];
        }
    }
#pragma unroll
    for (int i = 0; i < L; ++i) a[i] = max(lo[i], hi[L - 1 - i]);
    bitonic_sort_desc(a);
}

// The top-L keys of the wave's candidates (NC columns, k[c] for expert lane +
// 64 c) as one sorted list in every lane: each lane sorts its own, then six
// merges (xor 1, xor 2, rotate 4, rotate 8 within the row; row pairs;
// halves). Pick j is the j-th largest key r_j (0: nothing left); among the
// experts holding that key it is the (o + 1)-th lowest index, o the number of
// earlier picks with the same key -- the order of repeated strict-greater
// argmax passes. The picks' ballots are independent of each other, so the
// wave's dependent chain is the merge network alone.
template <int L, int NC, int KMAX>
__device__ __forceinline__ void topk_lists(const uint32_t (&k)[4], uint32_t TK,
                                           uint32_t (&pick)[KMAX], float (&chosen)[KMAX]) {
    uint32_t a[L];
#pragma unroll
    for (int i = 0; i < L; ++i) a[i] = 0u;
    if constexpr (NC == 2) {
        a[0] = max(k[0], k[1]);
        a[1] = min(k[0], k[1]);
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) a[c] = k[c];
        auto ce = [&](int i, int j) __attribute__((always_inline)) {
            const uint32_t x = a[i], y = a[j];
            a[i] = max(x, y);
            a[j] = min(x, y);
        };
        ce(0, 1), ce(2, 3), ce(0, 2), ce(1, 3), ce(1, 2);
    }
    list_merge_dpp<L, 0xB1>(a);   // quad_perm [1,0,3,2]
    list_merge_dpp<L, 0x4E>(a);   // quad_perm [2,3,0,1]
    list_merge_dpp<L, 0x124>(a);  // row_ror:4
    list_merge_dpp<L, 0x128>(a);  // row_ror:8
    list_merge_swap<L, false>(a);
    list_merge_swap<L, true>(a);
    uint32_t occ = 0, prev = 0;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
        pick[j] = 0;
        chosen[j] = -INFINITY;
        if (j >= L) continue;
        const uint32_t r = __builtin_amdgcn_readfirstlane(a[j]);
        occ = j > 0 && r == prev ? occ + 1 : 0u;
        prev = r;
        if ((uint32_t)j >= TK || r == 0u) continue;  // uniform
        uint64_t m[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) m[c] = __ballot(k[c] == r);
        for (uint32_t t = 0; t < occ; ++t) {  // uniform: drop the earlier picks of key r
            bool done = false;
#pragma unroll
            for (int c = 0; c < NC; ++c)
                if (!done && m[c] != 0ull) {
                    m[c] &= m[c] - 1ull;
                    done = true;
                }
        }
        uint32_t e = 0;
#pragma unroll
        for (int c = NC - 1; c >= 0; --c)
            if (m[c]) e = 64u * c + (uint32_t)__builtin_ctzll(m[c]);
        pick[j] = e;
        chosen[j] = key_value(r);
    }
}

// Top-k over one wave's candidates, v[q] = the logit of expert lane + 64 q (as
// cand() maps it), as the reference does it (moe-fused/src/kernels.metal:
// 149-156): pass j takes the largest remaining value -- the lowest index
// among equal values, as a strictly-greater ascending scan does -- and
// removes it; a pass with nothing selectable yields index 0 and -inf. Lists
// of 4 keys serve up to 4 picks, of 8 up to 8; columns 2 and 3 (experts
// 128-255) take part only when one of them holds a candidate. pick[] and
// chosen[] are uniform.
template <int KMAX>
__device__ __forceinline__ void topk_select(const float (&v)[4], uint32_t TK,
                                            uint32_t (&pick)[KMAX], float (&chosen)[KMAX]) {
    uint32_t k[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) k[q] = cand_key(v[q]);
    const bool wide = __ballot((k[2] | k[3]) != 0u) != 0;  // uniform
    if (TK <= 4) {
        if (wide) topk_lists<4, 4>(k, TK, pick, chosen);
        else topk_lists<4, 2>(k, TK, pick, chosen);
    } else {
        if (wide) topk_lists<8, 4>(k, TK, pick, chosen);
        else topk_lists<8, 2>(k, TK, pick, chosen);
    }
}

// SwiGLU of the reference (moe-fused/src/kernels.metal:177-215): the gate
// clamped above at 7, the up value to [-7, 7], alpha 1.702, (up + 1). The
// sigmoid's 1 / (1 + e) is the hardware reciprocal (v_rcp_f32, within 1 ulp):
// the correctly rounded form took ~10 more VALU per value, and every block
// form is issue-bound enough to feel it (0.2 / 0.4 / 1.3 us per block at
// 1 / 8 / 16 tokens, A/B in one process).
__device__ __forceinline__ float swiglu(float g, float u) {
    const float gg = fminf(g, 7.0f), uu = fminf(fmaxf(u, -7.0f), 7.0f);
    return gg * __builtin_amdgcn_rcpf(1.0f + __expf(-1.702f * gg)) * (uu + 1.0f);
}

}  // namespace kq
