// kq_device.h -- device helpers shared by the gfx950 kernels of libkq.
//
// Nibble -> fp16 without a convert instruction: OR-ing a 4-bit value into the
// mantissa of an fp16 constant gives an exact fp16 integer.
//   0x6400 is 1024.0 (ulp 1):    nibble in bits 0-3  -> 1024 + n
//   0x5400 is   64.0 (ulp 1/16): nibble in bits 4-7  ->   64 + n
// For one packed word w (nibble j = weight j) the four half2 operands
//   t0 = (w      & 0x000F000F) | 0x64006400  = (1024+n0, 1024+n4)
//   t1 = (w      & 0x00F000F0) | 0x54005400  = (  64+n1,   64+n5)
//   t2 = (w >> 8 & 0x000F000F) | 0x64006400  = (1024+n2, 1024+n6)
//   t3 = (w >> 8 & 0x00F000F0) | 0x54005400  = (  64+n3,   64+n7)
// cost one shift and four AND-OR ops per 8 weights. Dotted (fp32 accumulate)
// with the matching activation pairs (x0,x4) (x1,x5) (x2,x6) (x3,x7) they give
//   sum_j n_j x_j + 1024*(x0+x2+x4+x6) + 64*(x1+x3+x5+x7),
// and the constant term ("xc", per word or per chunk) depends on x only, so it
// is computed once per activation vector and subtracted per quant group.
// All products are exact in fp32 (11-bit x 11-bit significands).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kq {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr uint32_t kLo = 0x000F000Fu, kHi = 0x00F000F0u;
constexpr uint32_t kE1024 = 0x64006400u, kE64 = 0x54005400u;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ float bf2f(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Metadata element decode: KIND 0 = fp16, 1 = bf16.
template <int KIND>
__device__ __forceinline__ float meta2f(uint16_t v) {
    if constexpr (KIND == 1) return bf2f(v);
    else return h2f(v);
}

// ---- wave64 reductions on DPP (no LDS round trip) ----
// dpp_ctrl encodings (gfx9): quad_perm [1,0,3,2] = 0xB1 (xor 1),
// [2,3,0,1] = 0x4E (xor 2); row_ror:n = 0x120 + n; row_bcast:15 = 0x142,
// row_bcast:31 = 0x143.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 ROW_MASK, 0xF, false));
}
// Sum over each row of 16 lanes; every lane of the row gets its row's sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x124>(v);
    v += dpp_f<0x128>(v);
    return v;
}
// Sum over the 64 lanes of a wave, returned uniformly (from lane 63).
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    v += dpp_f<0x142, 0xA>(v);  // rows 1, 3 += lane 15 / 47
    v += dpp_f<0x143, 0xC>(v);  // rows 2, 3 += lane 31
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
// Sums over the two 32-lane halves of a wave: .x = lanes 0-31, .y = lanes 32-63.
__device__ __forceinline__ float2 half_sums(float v) {
    v = row16_sum(v);
    v += dpp_f<0x142, 0xA>(v);  // lane 31 = rows 0+1, lane 63 = rows 2+3
    return make_float2(
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 31)),
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63)));
}
// Sum over aligned groups of 4 lanes (every lane gets its group's sum).
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v;
}

// Permuted activation pairs of one 8-element word of x (fp16 bits, 4 dwords
// (x0,x1) (x2,x3) (x4,x5) (x6,x7)) -> (x0,x4) (x1,x5) (x2,x6) (x3,x7).
__device__ __forceinline__ u32x4 pair_perm(u32x4 v) {
    u32x4 p;
    p.x = (v.x & 0xFFFFu) | (v.z << 16);
    p.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
    p.z = (v.y & 0xFFFFu) | (v.w << 16);
    p.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
    return p;
}

// Plain sum and offset constant of one 8-element word of x (see header).
__device__ __forceinline__ void word_consts(u32x4 v, float& s, float& c) {
    float f0 = h2f(v.x & 0xFFFF), f1 = h2f(v.x >> 16), f2 = h2f(v.y & 0xFFFF), f3 = h2f(v.y >> 16);
    float f4 = h2f(v.z & 0xFFFF), f5 = h2f(v.z >> 16), f6 = h2f(v.w & 0xFFFF), f7 = h2f(v.w >> 16);
    float ev = (f0 + f4) + (f2 + f6), od = (f1 + f5) + (f3 + f7);
    s = ev + od;
    c = 1024.0f * ev + 64.0f * od;
}

// (a & b) | c. gfx9 VOP3 takes no literal operands, so with literal masks the
// compiler splits this into v_and + v_or; with b and c held in VGPRs whose
// values it cannot see (DequantConsts) it selects one v_and_or_b32. This stays
// plain C on purpose: the hazard recognizer does not model inline asm, and an
// asm VALU write into a register that an in-flight MFMA still reads as its A/B
// operand (WAR) gets no wait states.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t b, uint32_t c) {
    return (a & b) | c;
}

// The four dequant constants held in VGPRs.
struct DequantConsts {
    uint32_t lo, hi, e1024, e64;
    __device__ __forceinline__ DequantConsts() {
        // opaque to the optimiser so the values stay in VGPRs
        asm("v_mov_b32 %0, %1" : "=v"(lo) : "i"(kLo));
        asm("v_mov_b32 %0, %1" : "=v"(hi) : "i"(kHi));
        asm("v_mov_b32 %0, %1" : "=v"(e1024) : "i"(kE1024));
        asm("v_mov_b32 %0, %1" : "=v"(e64) : "i"(kE64));
    }
};

// The four fp16-pair operands of one packed word: (1024+n0, 1024+n4),
// (64+n1, 64+n5), (1024+n2, 1024+n6), (64+n3, 64+n7).
__device__ __forceinline__ u32x4 dq4(uint32_t w, const DequantConsts& k) {
    const uint32_t w8 = w >> 8;
    return u32x4{and_or(w, k.lo, k.e1024), and_or(w, k.hi, k.e64), and_or(w8, k.lo, k.e1024),
                 and_or(w8, k.hi, k.e64)};
}

// Dot of four dequantised pairs with their permuted activation pairs.
__device__ __forceinline__ float dot4(u32x4 d, u32x4 p, float acc) {
    acc = dot2(d.x, p.x, acc);
    acc = dot2(d.y, p.y, acc);
    acc = dot2(d.z, p.z, acc);
    return dot2(d.w, p.w, acc);
}

// Dot of one packed word (8 nibbles) with its permuted activation pairs.
__device__ __forceinline__ float qdot8(uint32_t w, u32x4 p, float acc, const DequantConsts& k) {
    const uint32_t w8 = w >> 8;
    acc = dot2(and_or(w, k.lo, k.e1024), p.x, acc);
    acc = dot2(and_or(w, k.hi, k.e64), p.y, acc);
    acc = dot2(and_or(w8, k.lo, k.e1024), p.z, acc);
    acc = dot2(and_or(w8, k.hi, k.e64), p.w, acc);
    return acc;
}

// Dot of one packed word with pairs (plain C; used where the register cost
// of the constants matters more than two instructions).
__device__ __forceinline__ float qdot8(uint32_t w, u32x4 p, float acc) {
    const uint32_t w8 = w >> 8;
    acc = dot2((w & kLo) | kE1024, p.x, acc);
    acc = dot2((w & kHi) | kE64, p.y, acc);
    acc = dot2((w8 & kLo) | kE1024, p.z, acc);
    acc = dot2((w8 & kHi) | kE64, p.w, acc);
    return acc;
}

// Raw buffer descriptor (stride 0; word 3 = the gfx9 default data format).
// Buffer loads address with a VGPR offset plus an SGPR offset; `bytes` is the
// range the hardware checks (< 2 GiB here).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
// Cache policies of buffer loads / stores: non-temporal (streamed weights);
// device-coherent (sc1: what agent-scope relaxed atomics use -- data shared
// between workgroups of one launch without an L2 write-back).
constexpr int kNT = 2;
constexpr int kSC1 = 16;

template <typename T>
__device__ __forceinline__ T ldg_nt(const T* p) {
    return __builtin_nontemporal_load(p);
}

}  // namespace kq
