// kq_int4_mfma_kernel.h -- int4 group-affine GEMV / skinny GEMM (batch <= 16)
// on the gfx950 matrix cores (v_mfma_f32_16x16x32_f16). Instantiated per
// quant-group size in kq_int4_mfma_g{32,64,128}.hip (compiled in parallel).
//
// Math (reference: int4-gemv/src/kernels.metal:17-31, 397-448):
//   y[b,m] = sum_g S[m,g] * (q[m,g,:] . x[b,g,:]) + B[m,g] * sum(x[b,g,:])
// Nibbles become fp16 by AND-OR into fp16 exponents (kq_device.h): a word
// gives (1024+n0,1024+n4)(64+n1,64+n5)(1024+n2,1024+n6)(64+n3,64+n7), so one
// word costs 1 shift + 4 AND-OR and the multiply-accumulate runs on the
// matrix pipe; the constant xc = 1024*sum(x_even) + 64*sum(x_odd) of a group
// is subtracted once per group in the epilogue acc += s*(D - xc) + b*xs.
//
// MFMA operands (D = A.B + C; A 16x32, B 32x16, measured lane layout):
//   A = x: lane l holds token l%16, 8 k of lane group g = l/16
//   B = W: lane l holds row   l%16, 8 k of lane group g     (one packed word)
//   D:     lane l holds tokens 4g+r (r < 4) of row l%16.
// Tokens beyond the batch hold zeros in A (their lanes never read x).
//
// Memory: a lane loads 16 B = words 4g..4g+3 of a 128-k "span" of its row,
// i.e. a wave instruction reads 64 B from each of 16 rows, and a wave streams
// consecutive spans of the same rows. Register j of lane group g then holds
// word 4g+j. For the per-group epilogue every MFMA's 32 k must lie in one
// quant group, which v_permlane{32,16}_swap arrange:
//   G = 128: one group per span, no exchange; MFMA j uses words 4g+j.
//   G = 64:  swap (r0,r2), (r1,r3) between lanes 0-31 and 32-63; registers
//            0,1 then hold group A (words 0-7), registers 2,3 group B.
//   G = 32:  a 4x4 transpose (the G = 64 swap, then permlane16 swaps of
//            (r0,r1), (r2,r3)); register j holds word 4j+g = group j.
// x is staged once per workgroup in LDS as permuted fp16 pairs, and each
// lane reads the words matching its (exchanged) registers.
//
// Work split: a 16-row tile is the unit of rows. A workgroup of P*Q waves
// owns a contiguous range of tiles; wave (p, q) takes K-part p (J = nspan/P
// consecutive spans) of tile q, q+Q, ... ("rounds"), and the P partial tiles
// of a round are summed in LDS in a fixed order (deterministic).
//
// Pipelining: each wave streams its (tile, span) steps through a ring of D
// register buffers. Every load is unconditional (out-of-range rows and steps
// are clamped to valid addresses and their results discarded) and is first
// used by the compute of its own step, so the waitcnt pass sees one straight
// sequence and waits for exactly one buffer at a time (vmcnt = loads of the
// other D-1 buffers). A branch around a load, or a use of loaded data right
// after the load, would make it wait for everything in flight.
#pragma once
#include "kq_device.h"
#include "kq_internal.h"

namespace kq {
namespace mfma {

constexpr int kMaxWaves = 16;
constexpr int kTile = 16;

struct Args {
    const uint32_t* W;
    const uint16_t* S;  // interleaved (scale, bias) pairs, or scales
    const uint16_t* B;  // biases (separate layout only)
    const uint16_t* X;  // [ntok][K] fp16
    void* Y;            // [ntok][M]
    uint32_t M, K, ntok, y_f32;
    uint32_t nspan, gpr;     // 128-k spans and quant groups per row
    uint32_t P, Q, J;        // K parts, tile lanes, spans per part
    uint32_t tiles_wg;       // tiles per workgroup (= rounds * Q)
    uint32_t ntiles;         // tiles in total
    uint32_t rounds;         // rounds per workgroup
    uint32_t nreal, nsteps;  // steps per wave (rounds * J) and padded to D
};

// Launch plan chosen on the host.
struct Plan {
    uint32_t P, Q, J, rounds, tiles_wg, nwg, nreal, nsteps, D, rmax;
    size_t lds;
};

// Scale/bias registers of one span (NG groups) as loaded, converted at use.
template <int NG, bool SB>
struct Meta;
template <int NG>
struct Meta<NG, true> {  // one dword (scale | bias << 16) per group
    uint32_t v[NG];
};
template <int NG>
struct Meta<NG, false> {  // NG scales and NG biases, two per dword
    uint32_t s[(NG + 1) / 2], b[(NG + 1) / 2];
};
template <>
struct Meta<1, false> {  // one scale, one bias: kept 16-bit until use
    uint16_t s[1], b[1];
};

template <int NG, bool SB>
struct Slot {
    u32x4 w;
    Meta<NG, SB> m;
};

template <int NG, bool SB>
__device__ __forceinline__ void load_meta(Meta<NG, SB>& m, const uint16_t* __restrict__ S,
                                          const uint16_t* __restrict__ B, size_t gi) {
    if constexpr (SB) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(S) + gi;
        if constexpr (NG == 1) {
            m.v[0] = *p;
        } else if constexpr (NG == 2) {
            const u32x2 t = *reinterpret_cast<const u32x2*>(p);
            m.v[0] = t.x;
            m.v[1] = t.y;
        } else {
            const u32x4 t = *reinterpret_cast<const u32x4*>(p);
            m.v[0] = t.x;
            m.v[1] = t.y;
            m.v[2] = t.z;
            m.v[3] = t.w;
        }
    } else {
        if constexpr (NG == 1) {
            m.s[0] = S[gi];
            m.b[0] = B[gi];
        } else if constexpr (NG == 2) {
            m.s[0] = *reinterpret_cast<const uint32_t*>(S + gi);
            m.b[0] = *reinterpret_cast<const uint32_t*>(B + gi);
        } else {
            const u32x2 s2 = *reinterpret_cast<const u32x2*>(S + gi);
            const u32x2 b2 = *reinterpret_cast<const u32x2*>(B + gi);
            m.s[0] = s2.x;
            m.s[1] = s2.y;
            m.b[0] = b2.x;
            m.b[1] = b2.y;
        }
    }
}

template <int NG, bool SB, bool BF>
__device__ __forceinline__ float2 meta_sb(const Meta<NG, SB>& m, int gg) {
    uint32_t sv, bv;
    if constexpr (SB) {
        sv = m.v[gg] & 0xFFFFu;
        bv = m.v[gg] >> 16;
    } else {
        const int h = (gg & 1) * 16;
        sv = (m.s[gg >> 1] >> h) & 0xFFFFu;
        bv = (m.b[gg >> 1] >> h) & 0xFFFFu;
    }
    if constexpr (BF) return make_float2(bf2f((uint16_t)sv), bf2f((uint16_t)bv));
    else return make_float2(h2f((uint16_t)sv), h2f((uint16_t)bv));
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

__device__ __forceinline__ f32x4 mfma(u32x4 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b, c, 0, 0, 0);
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

// LDS: xp [ntok][K/8] u32x4 | xk [ntok][K/G] float2 | part [2][waves][RMAX][64] f32
__host__ __device__ inline size_t lds_xp(uint32_t ntok, uint32_t K) { return (size_t)ntok * K * 2; }
__host__ __device__ inline size_t lds_xk(uint32_t ntok, uint32_t K, uint32_t G) {
    return (size_t)ntok * (K / G) * 8;
}
__host__ __device__ inline size_t lds_part(uint32_t waves, uint32_t rmax) {
    return (size_t)2 * waves * rmax * 64 * 4;
}

template <int GM, bool SB, bool BF, int RMAX, int D>
__global__ __launch_bounds__(1024) void int4_mfma(Args A) {
    constexpr int NG = 128 / GM;  // quant groups per span
    constexpr int WPG = GM / 8;   // words per group
    using SlotT = Slot<NG, SB>;

    extern __shared__ __align__(16) unsigned char smem[];
    const uint32_t K = A.K, nw = K >> 3, ngr = K / GM;
    u32x4* xp = reinterpret_cast<u32x4*>(smem);
    float2* xk = reinterpret_cast<float2*>(smem + lds_xp(A.ntok, K));
    float* part = reinterpret_cast<float*>(smem + lds_xp(A.ntok, K) + lds_xk(A.ntok, K, GM));

    const uint32_t tid = threadIdx.x, nthr = blockDim.x;
    const int lane = tid & 63;
    const uint32_t wave = tid >> 6;
    const uint32_t p = wave % A.P, q = wave / A.P;
    const uint32_t lrow = lane & 15, lg = lane >> 4;
    const uint32_t tile0 = blockIdx.x * A.tiles_wg;
    const uint32_t last_tile = A.ntiles - 1, last_row = A.M - 1;

    // ---- 1. first x staging loads (before any weight load: vmcnt is in order)
    const uint32_t xtotal = A.ntok * nw;
    const u32x4* X4 = reinterpret_cast<const u32x4*>(A.X);
    constexpr int kXr = 4;  // staging rounds per batch of loads
    u32x4 sv[kXr];
    auto x_load = [&](uint32_t w0) {
#pragma unroll
        for (int r = 0; r < kXr; ++r) {
            const uint32_t w = w0 + r * nthr + tid;
            sv[r] = X4[w < xtotal ? w : xtotal - 1];
        }
    };
    auto x_store = [&](uint32_t w0) {
#pragma unroll
        for (int r = 0; r < kXr; ++r) {
            const uint32_t w = w0 + r * nthr + tid;
            float s, c;
            word_consts(sv[r], s, c);
#pragma unroll
            for (int o = 1; o < WPG; o <<= 1) {
                s += __shfl_xor(s, o);
                c += __shfl_xor(c, o);
            }
            if (w < xtotal) {
                xp[w] = pair_perm(sv[r]);
                if (w % WPG == 0) xk[w / WPG] = make_float2(s, c);
            }
        }
    };
    x_load(0);
    // The scheduler may not interleave these loads: the loop's waits are
    // derived from the order they are issued in (also on entry to the loop).
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. prime the ring
    SlotT ring[D];
    auto issue = [&](SlotT& e, Cursor c) {
        if (c.round >= A.rounds) {  // padding step: re-read the last real one
            c.round = A.rounds - 1;
            c.j = A.J - 1;
        }
        const uint32_t tile = min(tile0 + c.round * A.Q + q, last_tile);
        const uint32_t row = min(tile * kTile + lrow, last_row);
        const uint32_t span = p * A.J + c.j;
        const u32x4* wp = reinterpret_cast<const u32x4*>(A.W + (size_t)row * nw + span * 16) + lg;
        e.w = ldg_nt(wp);
        load_meta<NG, SB>(e.m, A.S, A.B, (size_t)row * A.gpr + span * NG);
    };
    Cursor ci{0, 0};
#pragma unroll
    for (int d = 0; d < D; ++d) {
        issue(ring[d], ci);
        ci.advance(A.J);
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- 3. finish the x staging
    x_store(0);
    for (uint32_t w0 = kXr * nthr; w0 < xtotal; w0 += kXr * nthr) {
        x_load(w0);
        x_store(w0);
    }
    __syncthreads();

    // ---- 4. per-lane constants
    const DequantConsts kc;
    const bool has_tok = lrow < A.ntok;
    const u32x4* xrow = xp + (size_t)(has_tok ? lrow : 0) * nw;
    uint32_t xo[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xo[j] = xword<GM>(j, lg);
    const float2* xkr[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        const uint32_t t = min(4 * lg + r, A.ntok - 1);
        xkr[r] = xk + (size_t)t * ngr;
    }
    u32x4 xa[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) xa[j] = u32x4{0, 0, 0, 0};
    float acc[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) acc[r] = 0.0f;

    // ---- 5. one step: compute a slot, close the unit at the end of a part
    auto finish = [&](uint32_t round) {
        float* pw = part + (size_t)((round & 1) * (A.P * A.Q) + wave) * RMAX * 64;
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            pw[r * 64 + lane] = acc[r];
            acc[r] = 0.0f;
        }
        __syncthreads();
        const uint32_t per_tile = kTile * A.ntok, nout = A.Q * per_tile;
        const float* pr = part + (size_t)(round & 1) * (A.P * A.Q) * RMAX * 64;
        for (uint32_t i = tid; i < nout; i += nthr) {
            const uint32_t qq = i / per_tile, rem = i - qq * per_tile;
            const uint32_t t = rem >> 4, n = rem & 15;
            const uint32_t ls = 16 * (t >> 2) + n, r = t & 3;
            float v = 0.0f;
            for (uint32_t pp = 0; pp < A.P; ++pp)
                v += pr[(size_t)((qq * A.P + pp) * RMAX + r) * 64 + ls];
            const uint32_t tl = round * A.Q + qq, tile = tile0 + tl;
            const uint32_t row = tile * kTile + n;
            if (tl < A.tiles_wg && tile < A.ntiles && row < A.M) {
                const size_t o = (size_t)t * A.M + row;
                if (A.y_f32) reinterpret_cast<float*>(A.Y)[o] = v;
                else reinterpret_cast<uint16_t*>(A.Y)[o] = f2h(v);
            }
        }
    };
    auto step = [&](const SlotT& e, Cursor c, uint32_t n) {
        const uint32_t span = p * A.J + c.j;
        if (has_tok) {
            const u32x4* xs = xrow + span * 16;
#pragma unroll
            for (int j = 0; j < 4; ++j) xa[j] = xs[xo[j]];
        }
        uint32_t w[4] = {e.w.x, e.w.y, e.w.z, e.w.w};
        regroup<GM>(w);
        f32x4 dacc[NG];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            constexpr int per = 4 / NG;
            const int gg = j / per;
            const f32x4 cin = (j % per == 0) ? f32x4{0, 0, 0, 0} : dacc[gg];
            dacc[gg] = mfma(xa[j], dq(w[j], kc), cin);
        }
#pragma unroll
        for (int gg = 0; gg < NG; ++gg) {
            const float2 sb = meta_sb<NG, SB, BF>(e.m, gg);
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                const float2 k2 = xkr[r][span * NG + gg];
                acc[r] = fmaf(sb.x, dacc[gg][r] - k2.y, fmaf(sb.y, k2.x, acc[r]));
            }
        }
        if (n < A.nreal && c.j == A.J - 1) finish(c.round);
    };

    // ---- 6. main loop (loads D steps ahead), then the last D steps
    Cursor cc{0, 0};
    uint32_t n = 0;
    for (; n + D < A.nsteps; n += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            step(ring[d], cc, n + d);
            cc.advance(A.J);
            issue(ring[d], ci);
            ci.advance(A.J);
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        step(ring[d], cc, n + d);
        cc.advance(A.J);
    }
}

template <int GM, bool SB, bool BF, int RMAX, int D>
hipError_t go(const Args& a, const Plan& pl, hipStream_t s) {
    auto kern = int4_mfma<GM, SB, BF, RMAX, D>;
    if (pl.lds > 64 * 1024) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)pl.lds);
        if (e != hipSuccess) return e;
    }
    kern<<<pl.nwg, pl.P * pl.Q * 64, pl.lds, s>>>(a);
    return hipGetLastError();
}

template <int GM, bool SB, bool BF, int RMAX>
hipError_t go_d(const Args& a, const Plan& pl, hipStream_t s) {
    switch (pl.D) {
        case 2: return go<GM, SB, BF, RMAX, 2>(a, pl, s);
        case 4: return go<GM, SB, BF, RMAX, 4>(a, pl, s);
        case 8: return go<GM, SB, BF, RMAX, 8>(a, pl, s);
        default: return hipErrorInvalidValue;
    }
}

template <int GM>
hipError_t dispatch(const Args& a, const Plan& pl, bool sb, bool bf, hipStream_t s) {
#define KQ_R(SBV, BFV)                                                             \
    return pl.rmax == 1 ? go_d<GM, SBV, BFV, 1>(a, pl, s) : go_d<GM, SBV, BFV, 4>(a, pl, s)
    if (sb) {
        if (bf) KQ_R(true, true);
        KQ_R(true, false);
    }
    if (bf) KQ_R(false, true);
    KQ_R(false, false);
#undef KQ_R
}

}  // namespace mfma

hipError_t launch_mfma_g32(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                           hipStream_t s);
hipError_t launch_mfma_g64(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                           hipStream_t s);
hipError_t launch_mfma_g128(const mfma::Args& a, const mfma::Plan& pl, bool sb, bool bf,
                            hipStream_t s);

}  // namespace kq
