// kq_int4_mfma_kernel.h -- int4 group-affine skinny GEMM (1 to 16 tokens in
// one pass) on the gfx950 matrix cores. Instantiated per quant-group size in
// kq_int4_mfma_g{32,64,128}.hip (compiled in parallel).
//
// Math (reference: int4-gemv/src/kernels.metal:17-31, 397-448):
//   y[t,m] = sum_g S[m,g] * (q[m,g,:] . x[t,g,:]) + B[m,g] * sum(x[t,g,:])
// Nibbles become fp16 by AND-OR into fp16 exponents (kq_device.h): a word
// gives the eight values magic_k + q_k (magic 1024 or 64 by nibble parity),
// exact in fp16. Per quant group g the matrix cores form
//   Dg[t,m] = sum_{k in g} (magic_k + q_k) x[t,k]                (v_mfma 16x16x32 f16)
// and the epilogue is
//   acc[t,m] += S[m,g] * Dg[t,m]                                (VALU, 1 FMA per value)
//            +  sum_g ( B[m,g] * xs[t,g] + S[m,g] * xn[t,g] )    (v_mfma 16x16x4 f32)
// with xs = sum_{k in g} x_k and xn = -sum_{k in g} magic_k x_k. All products
// are exact in fp32 and every sum is an fp32 sum.
//
// xs and xn depend on x only. They come from one more f16 MFMA per 32 k whose
// A operand is a constant matrix (row 8w+p = ones over group 2p+w, row
// 8w+4+p = -magic over the same group, other rows zero) and whose B operand is
// the x registers the main MFMAs already hold. Its result lands with lane L
// holding, in register p, sum-row 4(L/16)+p of token L%16 -- exactly the A
// operand layout of v_mfma_f32_16x16x4_f32 (lane L: A[L%16][L/16]). So
// register p is the A operand of the correction MFMA for group pair p, whose
// B operand is (B, S, B', S') of the pair's two groups for row L%16 at k =
// L/16. No lane exchange is needed.
//
// MFMA operand layouts (D = A.B + C, measured):
//   16x16x32 f16: A lane L = row L%16, 8 k of group L/16; B lane L = column
//                 L%16, 8 k of group L/16; D lane L = rows 4(L/16)+r, col L%16.
//   x is A (rows = tokens), W is B (columns = weight rows), so D lane L holds
//   tokens 4(L/16)+r of weight row L%16; the accumulators keep that layout.
//
// Memory: an MFMA lane needs 16 B (4 words) of one row per 128-k "span", so
// a direct load would read 64 B from each of 16 rows per instruction -- an
// access shape that streams ~20% below the full rate. Weights are therefore
// loaded as span pairs: one instruction reads 128 B (two spans) from each of
// 8 rows (lane L: row L/8, 16-byte chunk L%8), two instructions per 16-row
// tile. The pair goes through a per-wave LDS stage of 16 rows x 128 B with
// the chunk index XOR-swizzled by the row (conflict-free writes and reads)
// and is read back in the MFMA operand layout, one span per step. x of the
// span comes with four 16-B loads per lane (L1/L2-resident), permuted in
// registers to the dequant order. All loads are buffer loads: the
// lane-constant part of an address sits in a VGPR and the span offset in an
// SGPR (or in the lane offset, where it must be range-checked), so
// addressing costs no vector instructions.
// For the per-group epilogue each MFMA's 32 k must lie in one quant group;
// v_permlane{32,16}_swap arrange that (G = 64: swap (r0,r2), (r1,r3) between
// the wave halves; G = 32: then permlane16 swaps of (r0,r1), (r2,r3)).
//
// Work split: a workgroup of P*Q waves owns groups_wg consecutive row groups
// (T tiles each); wave (p, q) takes K part p (J spans) of row groups q, q+Q,
// ... ("rounds"). The P partial tiles of a round are summed in LDS in a fixed
// order (deterministic).
//
// Scale/bias: loaded once per window of 8 spans (each lane holds two spans
// of its row; ds_bpermute hands a span's values to every lane of the row),
// since per-span loads of 2-16 bytes from 16 rows cost more than the weights.
//
// Pipelining: each wave streams its (row group, span) steps through a ring of
// D register slots (ring_depth: 4 at two tiles a wave, else 2; an even slot
// also holds its span pair's weights). Every load is unconditional: rows past the end are
// clamped to valid addresses (results discarded), and padding steps (a part
// padded to whole windows of 8 spans) load out
// of the descriptors' range -- zeros, which add exactly nothing, and no
// memory traffic. Each load is first used by the compute of its own step, so
// the waitcnt pass sees one straight sequence and waits for exactly one slot
// at a time.
#pragma once
#include <type_traits>

#include "kq_device.h"
#include "kq_internal.h"

namespace kq {
namespace mfma {

constexpr int kTile = 16;

struct Args {
    const uint32_t* W;
    const uint16_t* S;  // interleaved (scale, bias) pairs, or scales
    const uint16_t* B;  // biases (separate layout only)
    const uint16_t* X;  // [ntok][K] fp16
    void* Y;            // [ntok][M]
    uint32_t M, K, ntok, y_f32;
    uint32_t gpr;                // quant groups per row
    uint32_t P, Q, J, J8;        // K parts, row-group lanes, spans per part (J8: padded to windows)
    uint32_t ngroups;            // row groups (T tiles each) in total
    uint32_t groups_wg, rounds;  // row groups per workgroup (= rounds * Q)
    uint32_t nsteps;             // steps per wave (rounds * J8: whole windows)
    uint32_t part_bytes;         // LDS of the K-part reduction (the weight staging follows)
};

// Launch plan chosen on the host.
struct Plan {
    uint32_t T, P, Q, J, J8, rounds, groups_wg, nwg, nsteps, waves;
    size_t lds;
};

// Waves per workgroup that the register budget of (G, T, D) allows without
// spills: 16 waves leave 128 registers per lane, 8 leave 256.
__host__ __device__ constexpr uint32_t max_waves(uint32_t G, uint32_t T) {
    return T >= 2 || G == 32 ? 8 : 16;
}

// Ring depth in steps (even: a step pair shares one weight load). Two tiles
// a wave have the registers for two span pairs ahead (198 VGPRs of 256);
// four tiles (202 at depth 2) and one tile at 16 waves (116 of 128) do not.
// Depth 4 at two tiles, with the planner counting its loads in flight:
// 8192x28672 at 16 tokens 42.3 -> 40.6 us, 14336x4096 26.5 -> 20.1 us.
__host__ __device__ constexpr int ring_depth(uint32_t T) { return T == 2 ? 4 : 2; }

__host__ __device__ inline size_t lds_part(uint32_t waves, uint32_t T, uint32_t rounds, uint32_t P) {
    return P > 1 ? (size_t)(rounds > 1 ? 2 : 1) * waves * T * 4 * 64 * 4 : 0;
}
// Per wave: the span-pair staging of its T tiles (16 rows x 128 bytes each).
__host__ __device__ inline size_t lds_wstage(uint32_t waves, uint32_t T) {
    return (size_t)waves * T * 2048;
}


// Scale/bias registers of one span (NG groups), converted at use.
template <int NG, bool SB>
struct Meta;
// (Vector types, not arrays: an array member of the ring's slots can keep the
// whole ring out of registers.)
template <>
struct Meta<1, true> {  // one dword (scale | bias << 16) per group
    uint32_t v;
};
template <>
struct Meta<2, true> {
    u32x2 v;
};
template <>
struct Meta<4, true> {
    u32x4 v;
};
template <int NG>
__device__ __forceinline__ uint32_t mword(const Meta<NG, true>& m, int gi) {
    if constexpr (NG == 1) return m.v;
    else return m.v[gi];
}
template <>
struct Meta<1, false> {  // one scale, one bias: kept 16-bit until use
    uint16_t s, b;
};
template <>
struct Meta<2, false> {  // two scales, two biases, one dword each
    uint32_t s, b;
};
template <>
struct Meta<4, false> {
    u32x2 s, b;
};

// Low 16 bits of `raw` as a float (fp16 or bf16 bits).
template <bool BF>
__device__ __forceinline__ float lo16f(uint32_t raw) {
    if constexpr (BF) return __builtin_bit_cast(float, raw << 16);
    else return (float)__builtin_bit_cast(_Float16, (uint16_t)raw);
}

// Scale of group gi for this lane's row.
template <int NG, bool SB, bool BF>
__device__ __forceinline__ float sval(const Meta<NG, SB>& m, int gi) {
    uint32_t raw;
    if constexpr (SB) raw = mword<NG>(m, gi);
    else if constexpr (NG == 1) raw = m.s;
    else if constexpr (NG == 2) raw = gi ? m.s >> 16 : m.s;
    else raw = (gi & 1) ? m.s[gi >> 1] >> 16 : m.s[gi >> 1];
    return lo16f<BF>(raw);
}

// B operand of the correction MFMA of group pair p for lane group kg:
// kg = 0: bias of group 2p, 1: scale of 2p, 2: bias of 2p+1, 3: scale of 2p+1
// (zero where the group does not exist). shs = 16 for biases, 0 for scales
// (interleaved dwords); hsel = 16 * (kg >> 1) (separate arrays).
template <int NG, bool SB, bool BF>
__device__ __forceinline__ float bcorr(const Meta<NG, SB>& m, int p, bool hi_grp, bool want_s,
                                       uint32_t shs, uint32_t hsel) {
    uint32_t raw;
    if constexpr (SB) {
        uint32_t d;
        if constexpr (NG == 1) d = hi_grp ? 0u : m.v;
        else d = hi_grp ? m.v[2 * p + 1] : m.v[2 * p];
        raw = d >> shs;
    } else if constexpr (NG == 1) {
        const uint32_t d = want_s ? (uint32_t)m.s : (uint32_t)m.b;
        raw = hi_grp ? 0u : d;
    } else if constexpr (NG == 2) {
        raw = (want_s ? m.s : m.b) >> hsel;
    } else {
        raw = (want_s ? m.s[p] : m.b[p]) >> hsel;
    }
    return lo16f<BF>(raw);
}

// Word (of the span's 16) that register j of lane group g holds after regroup.
template <int GM>
__device__ __forceinline__ uint32_t xword(int j, uint32_t g) {
    if constexpr (GM == 128) return 4 * g + j;
    else if constexpr (GM == 64) return (g & 1) * 4 + (g >> 1) * 2 + (j & 1) + (j >> 1) * 8;
    else return 4 * j + g;
}

template <int GM>
__device__ __forceinline__ void regroup(uint32_t (&w)[4]) {
    if constexpr (GM == 64 || GM == 32) {
        const auto a = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
        const auto b = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
        w[0] = a[0];
        w[2] = a[1];
        w[1] = b[0];
        w[3] = b[1];
    }
    if constexpr (GM == 32) {
        const auto a = __builtin_amdgcn_permlane16_swap(w[0], w[1], false, false);
        const auto b = __builtin_amdgcn_permlane16_swap(w[2], w[3], false, false);
        w[0] = a[0];
        w[1] = a[1];
        w[2] = b[0];
        w[3] = b[1];
    }
}

__device__ __forceinline__ f16x8 dq(uint32_t w, const DequantConsts& k) {
    const uint32_t w8 = w >> 8;
    const u32x4 t{and_or(w, k.lo, k.e1024), and_or(w, k.hi, k.e64), and_or(w8, k.lo, k.e1024),
                  and_or(w8, k.hi, k.e64)};
    return __builtin_bit_cast(f16x8, t);
}

// x pairs (x0,x1)(x2,x3)(x4,x5)(x6,x7) -> dequant order (x0,x4)(x1,x5)(x2,x6)(x3,x7).
__device__ __forceinline__ f16x8 xperm(u32x4 v) {
    const u32x4 p{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                  __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
    return __builtin_bit_cast(f16x8, p);
}

__device__ __forceinline__ f32x4 mma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Position of a wave in its (round, span) sequence.
struct Cursor {
    uint32_t j, round;
    __device__ __forceinline__ void advance(uint32_t J) {
        if (++j == J) {
            j = 0;
            ++round;
        }
    }
};

// Scale/bias of a window of kWin spans as loaded: lane (row n, group kg)
// holds spans 2kg, 2kg + 1 of the window, so one instruction reads 8 spans'
// worth of each of 16 rows (32-128 contiguous bytes per row, instead of 2-16
// per span). At each span the values are fetched from the owning lane with
// ds_bpermute (no LDS allocation).
constexpr int kWin = 8;
template <int NG, bool SB>
struct MWin;
template <>
struct MWin<1, true> {
    u32x2 a;  // 2 spans x 1 dword
};
template <>
struct MWin<2, true> {
    u32x4 a;  // 2 spans x 2 dwords
};
template <>
struct MWin<4, true> {
    u32x4 a, c;  // span 0, span 1: 4 dwords each
};
template <>
struct MWin<1, false> {
    uint32_t s, b;  // 2 spans x 1 half
};
template <>
struct MWin<2, false> {
    u32x2 s, b;  // 2 spans x 2 halves
};
template <>
struct MWin<4, false> {
    u32x4 s, b;  // 2 spans x 4 halves
};

template <int NG, bool SB>
__device__ __forceinline__ void load_mwin(MWin<NG, SB>& m, rsrc_t rs, rsrc_t rb, uint32_t vo) {
    if constexpr (SB) {
        if constexpr (NG == 1) m.a = __builtin_amdgcn_raw_buffer_load_b64(rs, vo, 0, 0);
        else if constexpr (NG == 2) m.a = __builtin_amdgcn_raw_buffer_load_b128(rs, vo, 0, 0);
        else {
            m.a = __builtin_amdgcn_raw_buffer_load_b128(rs, vo, 0, 0);
            m.c = __builtin_amdgcn_raw_buffer_load_b128(rs, vo + 16, 0, 0);
        }
    } else if constexpr (NG == 1) {
        m.s = __builtin_amdgcn_raw_buffer_load_b32(rs, vo, 0, 0);
        m.b = __builtin_amdgcn_raw_buffer_load_b32(rb, vo, 0, 0);
    } else if constexpr (NG == 2) {
        m.s = __builtin_amdgcn_raw_buffer_load_b64(rs, vo, 0, 0);
        m.b = __builtin_amdgcn_raw_buffer_load_b64(rb, vo, 0, 0);
    } else {
        m.s = __builtin_amdgcn_raw_buffer_load_b128(rs, vo, 0, 0);
        m.b = __builtin_amdgcn_raw_buffer_load_b128(rb, vo, 0, 0);
    }
}

__device__ __forceinline__ uint32_t bperm(uint32_t addr, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_ds_bpermute((int)addr, (int)v);
}

// Meta of window span R for this lane's row; ba = 4 * (n + 16 * (R / 2)).
template <int NG, bool SB, int R>
__device__ __forceinline__ Meta<NG, SB> meta_at(const MWin<NG, SB>& w, uint32_t ba) {
    constexpr int SUB = R & 1;
    Meta<NG, SB> m;
    if constexpr (SB) {
        if constexpr (NG == 1) m.v = bperm(ba, SUB ? w.a.y : w.a.x);
        else if constexpr (NG == 2) m.v = u32x2{bperm(ba, w.a[2 * SUB]), bperm(ba, w.a[2 * SUB + 1])};
        else {
            const u32x4 src = SUB ? w.c : w.a;
            m.v = u32x4{bperm(ba, src.x), bperm(ba, src.y), bperm(ba, src.z), bperm(ba, src.w)};
        }
    } else if constexpr (NG == 1) {
        m.s = (uint16_t)(bperm(ba, w.s) >> (16 * SUB));
        m.b = (uint16_t)(bperm(ba, w.b) >> (16 * SUB));
    } else if constexpr (NG == 2) {
        m.s = bperm(ba, w.s[SUB]);
        m.b = bperm(ba, w.b[SUB]);
    } else {
        m.s = u32x2{bperm(ba, w.s[2 * SUB]), bperm(ba, w.s[2 * SUB + 1])};
        m.b = u32x2{bperm(ba, w.b[2 * SUB]), bperm(ba, w.b[2 * SUB + 1])};
    }
    return m;
}

// Ring slots. Even steps also carry the weights of a span pair: per tile two
// loads of 8 rows x 128 contiguous bytes (a lane: row 8h + l/8, 16-byte
// chunk (l % 8) ^ (row % 8) of the pair).
template <int T>
struct SlotE {
    u32x4 w[T][2];
    u32x4 x[4];
};
struct SlotO {
    u32x4 x[4];
};

template <int F, typename Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
    if constexpr (F > 0) {
        static_for<F - 1>(f);
        f(std::integral_constant<int, F - 1>{});
    }
}

template <int GM, bool SB, bool BF, int T, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void int4_mfma(Args A) {
    constexpr int NG = 128 / GM;         // quant groups per span
    constexpr int NP = (NG + 1) / 2;     // group pairs (correction MFMAs) per span
    constexpr int PER = 4 / NG;          // MFMAs per group
    constexpr uint32_t MB = SB ? 4 : 2;  // meta bytes per group (per array)
    constexpr int D = ring_depth(T);     // ring depth (steps)
    constexpr int U = kWin;              // steps per loop body (one meta window)


    extern __shared__ __align__(16) unsigned char smem[];
    float* part = reinterpret_cast<float*>(smem);

    const uint32_t K = A.K, M = A.M;
    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    // the wave index is uniform; say so, or every buffer load whose scalar
    // offset derives from it becomes a waterfall loop
    const uint32_t lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t p = wave % A.P, q = wave / A.P;
    const uint32_t n = lane & 15, kg = lane >> 4;
    const uint32_t g0 = blockIdx.x * A.groups_wg;
    // this wave's span-pair staging: per tile 16 rows x 128 bytes (swizzled)
    unsigned char* wst = smem + A.part_bytes + (size_t)wave * T * 2048;

    const rsrc_t rW = make_rsrc(A.W, M * (K / 2));
    const rsrc_t rS = make_rsrc(A.S, M * A.gpr * MB);
    const rsrc_t rB = make_rsrc(SB ? A.S : A.B, M * A.gpr * MB);
    const rsrc_t rX = make_rsrc(A.X, A.ntok * K * 2);
    constexpr uint32_t kOOB = 0x80000000u;  // past every descriptor's range: the load reads zeros

    // lane-constant parts of the x addresses (token n, clamped into the batch)
    uint32_t xvo[4];
    {
        const uint32_t t = n < A.ntok ? n : A.ntok - 1;
#pragma unroll
        for (int j = 0; j < 4; ++j) xvo[j] = t * K * 2 + xword<GM>(j, kg) * 16;
    }
    uint32_t ba[4];  // ds_bpermute addresses of lane (n, group k)
#pragma unroll
    for (int k = 0; k < 4; ++k) ba[k] = 4 * (n + 16 * k);

    // LDS read offsets of (row n, chunk 4s + kg) for span s of a pair
    uint32_t rdo[2];
#pragma unroll
    for (int sp = 0; sp < 2; ++sp)
        rdo[sp] = (n >> 3) * 1024 + ((((n & 7) << 3) | ((4 * sp + kg) ^ (n & 7))) * 16);

    // lane-constant parts of the weight / meta addresses of the current issue round
    uint32_t wvo[T][2], mvo[T];
    uint32_t cur_rg = 0xFFFFFFFFu;
    auto set_rows = [&](uint32_t rg) __attribute__((always_inline)) {
        cur_rg = rg;
#pragma unroll
        for (int i = 0; i < T; ++i) {
            uint32_t row = rg * (16 * T) + 16 * i + n;
            row = row < M ? row : M - 1;
            mvo[i] = row * A.gpr * MB;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t r = rg * (16 * T) + 16 * i + 8 * h + (lane >> 3);
                r = r < M ? r : M - 1;
                wvo[i][h] = r * (K / 2) + (((lane & 7) ^ ((lane >> 3) & 7)) * 16);
            }
        }
    };

    // ---- the load stream. Steps past a part's J spans (padding to whole
    // windows) and past the last round load out of range: zeros, which add
    // nothing (x = 0 and scale/bias = 0), and cost no memory traffic.
    // named buffers, not arrays: arrays of these (selected by constant
    // indices after unrolling) have been kept in scratch by the compiler
    SlotE<T> ring0, ring2;
    SlotO ring1, ring3;
    // scale/bias windows: mwb receives the next window's loads, mwa holds the
    // current one (copied from mwb at the window's first step)
    MWin<NG, SB> mwa[T], mwb[T];
    auto slot = [&](auto k) __attribute__((always_inline)) -> auto& {
        constexpr int kk = decltype(k)::value;
        if constexpr (kk == 0) return ring0;
        else if constexpr (kk == 1) return ring1;
        else if constexpr (kk == 2) return ring2;
        else return ring3;
    };
    auto issue = [&](auto& e, Cursor c, auto win) __attribute__((always_inline)) {
        const bool ok = c.round < A.rounds && c.j < A.J;
        uint32_t rg = g0 + (c.round < A.rounds ? c.round : A.rounds - 1) * A.Q + q;
        rg = __builtin_amdgcn_readfirstlane(rg < A.ngroups ? rg : A.ngroups - 1);
        if (rg != cur_rg) set_rows(rg);
        // uniform by construction; readfirstlane keeps it in an SGPR (a scalar
        // offset the compiler thinks divergent becomes a waterfall loop)
        const uint32_t span = __builtin_amdgcn_readfirstlane(p * A.J + (c.j < A.J ? c.j : A.J - 1));
        const uint32_t oob = ok ? 0u : kOOB;
        if constexpr (decltype(win)::value >= 0) {  // first step of a window: its scale/bias
            const uint32_t j2 = c.j + 2 * kg;
            const bool lok = c.round < A.rounds && j2 < A.J;
            const uint32_t lspan = p * A.J + (j2 < A.J ? j2 : A.J - 1);
#pragma unroll
            for (int i = 0; i < T; ++i)
                load_mwin<NG, SB>(mwb[i], rS, rB,
                                  mvo[i] + lspan * NG * MB + (lok ? 0u : kOOB));
        }
        if constexpr (std::is_same_v<std::decay_t<decltype(e)>, SlotE<T>>) {
            // the pair (span, span + 1); its offset goes in the lane offset, so
            // the range check covers a pair running past the last row
            const uint32_t po = span * 64 + oob;
#pragma unroll
            for (int i = 0; i < T; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    e.w[i][h] = __builtin_amdgcn_raw_buffer_load_b128(rW, wvo[i][h] + po, 0, kNT);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
            e.x[j] = __builtin_amdgcn_raw_buffer_load_b128(rX, xvo[j] + oob, span * 256, 0);
    };
    Cursor ci{0, 0};
    static_for<D>([&](auto kk) __attribute__((always_inline)) {
        constexpr int k = decltype(kk)::value;
        issue(slot(kk), ci, std::integral_constant<int, k % kWin == 0 ? 0 : -1>{});
        ci.advance(A.J8);
        __builtin_amdgcn_sched_barrier(0);
    });

    // ---- per-lane constants
    const DequantConsts kc;
    // constant A operands of the sums MFMA, one per group of the span
    f16x8 ac[NG];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        const uint32_t rs = 8 * (gi & 1) + (gi >> 1), rc = rs + 4;
        const u32x4 ones{0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
        const u32x4 negm{0xE400E400u, 0xD400D400u, 0xE400E400u, 0xD400D400u};
        const u32x4 zero{0u, 0u, 0u, 0u};
        ac[gi] = __builtin_bit_cast(f16x8, n == rs ? ones : n == rc ? negm : zero);
    }
    const bool hi_grp = kg >= 2, want_s = (kg & 1) != 0;
    const uint32_t shs = want_s ? 0u : 16u, hsel = hi_grp ? 16u : 0u;
    f32x4 acc[T];
#pragma unroll
    for (int i = 0; i < T; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // ---- close a round: sum the P parts (LDS, fixed order) and store y
    auto store = [&](uint32_t row, uint32_t t, float v) {
        if (t < A.ntok && row < M) {
            const size_t o = (size_t)t * M + row;
            if (A.y_f32) reinterpret_cast<float*>(A.Y)[o] = v;
            else reinterpret_cast<uint16_t*>(A.Y)[o] = f2h(v);
        }
    };
    auto finish = [&](uint32_t round) {
        const uint32_t rgw = g0 + round * A.Q;  // first row group of this round in the workgroup
        if (A.P == 1) {
            const uint32_t rg = rgw + q;
            if (rg < A.ngroups) {
#pragma unroll
                for (int i = 0; i < T; ++i)
#pragma unroll
                    for (int r = 0; r < 4; ++r) store(rg * (16 * T) + 16 * i + n, 4 * kg + r, acc[i][r]);
            }
        } else {
            float* pw = part + ((size_t)((A.rounds > 1 ? (round & 1) : 0) * (A.P * A.Q) + wave) * T) * 256;
#pragma unroll
            for (int i = 0; i < T; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) pw[(i * 4 + r) * 64 + lane] = acc[i][r];
            __syncthreads();
            const float* pr = part + (size_t)((A.rounds > 1 ? (round & 1) : 0) * (A.P * A.Q)) * T * 256;
            const uint32_t per_grp = T * 16 * A.ntok, nout = A.Q * per_grp;
            for (uint32_t o = tid; o < nout; o += nthr) {
                const uint32_t qq = o / per_grp, rem = o - qq * per_grp;
                const uint32_t i = rem / (16 * A.ntok), rem2 = rem - i * 16 * A.ntok;
                const uint32_t t = rem2 >> 4, nn = rem2 & 15;
                const uint32_t ls = 16 * (t >> 2) + nn, r = t & 3;
                float v = 0.0f;
                for (uint32_t pp = 0; pp < A.P; ++pp) v += pr[((size_t)(qq * A.P + pp) * T * 4 + i * 4 + r) * 64 + ls];
                const uint32_t rg = rgw + qq;
                if (rg < A.ngroups) store(rg * (16 * T) + 16 * i + nn, t, v);
            }
        }
#pragma unroll
        for (int i = 0; i < T; ++i) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };

    // ---- one step: x-only sums, then per tile the group MFMAs and epilogue.
    // RW = the step's span within its window.
    auto step = [&](const auto& e, Cursor c, auto rw) __attribute__((always_inline)) {
        constexpr int RW = decltype(rw)::value, SP = RW & 1;
        if constexpr (RW == 0) {
#pragma unroll
            for (int i = 0; i < T; ++i) mwa[i] = mwb[i];
        }
        if constexpr (SP == 0) {  // stage the pair's weights in LDS (this wave's area)
#pragma unroll
            for (int i = 0; i < T; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    *reinterpret_cast<u32x4*>(wst + i * 2048 + h * 1024 + lane * 16) = e.w[i][h];
        }
        f16x8 xa[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) xa[j] = xperm(e.x[j]);
        // Phases over all tiles, so that each tile's MFMA results are not
        // read until the other tiles' dequant and MFMAs have been issued:
        // LDS reads and meta, then dequant + group MFMAs, then epilogues.
        u32x4 wv[T];
        Meta<NG, SB> m[T];
#pragma unroll
        for (int i = 0; i < T; ++i) {
            wv[i] = *reinterpret_cast<const u32x4*>(wst + i * 2048 + rdo[SP]);
            m[i] = meta_at<NG, SB, RW>(mwa[i], ba[RW / 2]);
        }
        f32x4 sums{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) sums = mma16(ac[j / PER], xa[j], sums);
        f32x4 dg[T][NG];
        // tile e's epilogue follows tile e + S's MFMAs; S = T - 1 measured
        // best (S = 0, 1 and T - 1 compared; 1-3% over S = 0)
        constexpr int S = T - 1;
        static_for<T + S>([&](auto ii) __attribute__((always_inline)) {
            constexpr int i = decltype(ii)::value;
            if constexpr (i < T) {
                uint32_t w[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
                regroup<GM>(w);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int gi = j / PER;
                    const f32x4 cin = (j % PER == 0) ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : dg[i][gi];
                    dg[i][gi] = mma16(xa[j], dq(w[j], kc), cin);
                }
            }
            if constexpr (i >= S) {
                constexpr int e = i - S;
#pragma unroll
                for (int gi = 0; gi < NG; ++gi) {
                    const float sc = sval<NG, SB, BF>(m[e], gi);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[e][r] = fmaf(sc, dg[e][gi][r], acc[e][r]);
                }
#pragma unroll
                for (int pp = 0; pp < NP; ++pp)
                    acc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        sums[pp], bcorr<NG, SB, BF>(m[e], pp, hi_grp, want_s, shs, hsel), acc[e], 0, 0, 0);
            }
        });
        if (c.round < A.rounds && c.j == A.J8 - 1) finish(c.round);
    };

    // ---- main loop: one meta window per body (every buffer index is a
    // constant), loads D steps ahead; then the last window
    Cursor cc{0, 0};
    uint32_t ns = 0;
    for (; ns + U < A.nsteps; ns += U) {
        static_for<U>([&](auto dd) __attribute__((always_inline)) {
            constexpr int d = decltype(dd)::value;
            step(slot(std::integral_constant<int, d % D>{}), cc, std::integral_constant<int, d>{});
            cc.advance(A.J8);
            constexpr int nx = d + D;  // the step issued now, relative to ns
            issue(slot(std::integral_constant<int, d % D>{}), ci,
                  std::integral_constant<int, nx % kWin == 0 ? 0 : -1>{});
            ci.advance(A.J8);
        });
    }
    static_for<U>([&](auto dd) __attribute__((always_inline)) {
        constexpr int d = decltype(dd)::value;
        step(slot(std::integral_constant<int, d % D>{}), cc, std::integral_constant<int, d>{});
        cc.advance(A.J8);
        if constexpr (d + D < U) {
            issue(slot(std::integral_constant<int, d % D>{}), ci, std::integral_constant<int, -1>{});
            ci.advance(A.J8);
        }
    });
}

template <int GM, bool SB, bool BF, int T, int WAVES>
hipError_t go(const Args& a, const Plan& pl, hipStream_t s) {
    auto kern = int4_mfma<GM, SB, BF, T, WAVES>;
    if (pl.lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)pl.lds);
        if (e != hipSuccess) return e;
    }
    kern<<<pl.nwg, pl.waves * 64, pl.lds, s>>>(a);
    return hipGetLastError();
}

template <int GM, bool SB, bool BF>
hipError_t go_td(const Args& a, const Plan& pl, hipStream_t s) {
    if (pl.T == 4) return go<GM, SB, BF, 4, max_waves(GM, 4)>(a, pl, s);
    if (pl.T == 2) return go<GM, SB, BF, 2, max_waves(GM, 2)>(a, pl, s);
    if (pl.T == 1) return go<GM, SB, BF, 1, max_waves(GM, 1)>(a, pl, s);
    return hipErrorInvalidValue;
}

template <int GM>
hipError_t dispatch(const Args& a, const Plan& pl, bool sb, bool bf, hipStream_t s) {
    if (sb) return bf ? go_td<GM, true, true>(a, pl, s) : go_td<GM, true, false>(a, pl, s);
    return bf ? go_td<GM, false, true>(a, pl, s) : go_td<GM, false, false>(a, pl, s);
}

}  // namespace mfma

hipError_t launch_mfma_g32(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                           hipStream_t s);
hipError_t launch_mfma_g64(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                           hipStream_t s);
hipError_t launch_mfma_g128(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                            hipStream_t s);

}  // namespace kq
