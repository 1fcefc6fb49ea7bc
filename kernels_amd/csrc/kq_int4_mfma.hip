// kq_int4_mfma.hip -- launch planning for the matrix-core int4 path (the
// kernel is in kq_int4_mfma_kernel.h, instantiated per quant-group size in
// kq_int4_mfma_g{32,64,128}.hip).
//
// A plan fixes the tiles per wave T (4 with at most 8 waves per workgroup, 2
// or 1 with at most 16: the register budget of T), the split of a
// workgroup's waves into P K-parts (P divides the number of 128-k spans) and
// Q row-group lanes (Q cut to the row groups a CU has) and the row groups per
// workgroup (in rounds of Q).
// Cost = the busiest CU's weight bytes (workgroups it runs x waves x padded
// steps x T), times a latency factor when a CU has less than ~48 KiB of loads
// in flight. All tokens (up to 16) go in one pass.
#include "kq_int4_mfma_kernel.h"

namespace kq {

namespace {


constexpr size_t kLdsMax = 160 * 1024;

bool make_plan(uint32_t M, uint32_t K, uint32_t G, uint32_t ntok, Int4Cfg cfg, mfma::Plan& out) {
    (void)ntok;
    const uint32_t nspan = K / 128, ntiles = (M + mfma::kTile - 1) / mfma::kTile, cu = cu_count();
    // cfg.unroll: 0 = automatic, or 10 * T + T's ring depth (12, 24, 42);
    // cfg.rows: K parts P (0 = automatic)
    uint32_t fT = 0;
    if (cfg.unroll != 0) {
        fT = (uint32_t)cfg.unroll / 10;
        if (cfg.unroll < 0 || (fT != 1 && fT != 2 && fT != 4) ||
            (uint32_t)cfg.unroll % 10 != (uint32_t)mfma::ring_depth(fT))
            return false;
    }
    bool found = false;
    double best = 0.0;
    for (uint32_t T : {4u, 2u, 1u}) {
        if (fT && T != fT) continue;
        const uint32_t wmax = mfma::max_waves(G, T);
        const uint32_t ngroups = (ntiles + T - 1) / T;
        for (uint32_t P = 1; P <= wmax; ++P) {
            if (nspan % P) continue;
            if (cfg.rows > 0 && (uint32_t)cfg.rows != P) continue;
            // Q is cut to the row groups a CU has (no idle lanes)
            const uint32_t qmax = wmax / P, J = nspan / P;
            const uint32_t J8 = (J + mfma::kWin - 1) / mfma::kWin * mfma::kWin;
            const uint32_t per_cu = (ngroups + cu - 1) / cu;
            const uint32_t rounds = (per_cu + qmax - 1) / qmax;
            const uint32_t Q = (per_cu + rounds - 1) / rounds, waves = P * Q;
            const uint32_t groups_wg = rounds * Q;
            const uint32_t nwg = (ngroups + groups_wg - 1) / groups_wg;
            const uint32_t nsteps = rounds * J8;  // whole windows (the loop body is one)
            const size_t lds = mfma::lds_part(waves, T, rounds, P) + mfma::lds_wstage(waves, T);
            if (lds > kLdsMax) continue;
            // padding steps move no bytes but take issue slots
            const double steps = rounds * J + 0.3 * (nsteps - rounds * J);
            // KiB per CU: D/2 span pairs of T 2-KiB tiles per wave
            const double inflight = (double)waves * mfma::ring_depth(T) * T;
            const double cost = (double)((nwg + cu - 1) / cu) * waves * steps * T *
                                (inflight < 48.0 ? 48.0 / inflight : 1.0) * (P > 1 ? 1.02 : 1.0);
            if (!found || cost < best) {
                found = true;
                best = cost;
                out = mfma::Plan{T, P, Q, J, J8, rounds, groups_wg, nwg, nsteps, waves, lds};
            }
        }
    }
    return found;
}

}  // namespace

uint32_t int4_mfma_tokens_per_pass(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg) {
    mfma::Plan pl;
    return int4_mfma_supported(M, K, G, batch, cfg) && make_plan(M, K, G, batch, cfg, pl) ? batch : 0;
}

// The pass is bound by each wave's serial steps (dequant, MFMA chains,
// epilogue), not by HBM at these sizes: ~0.42 us per (step x tile) at 8 waves
// a CU, plus ~3.3 us of launch and ramp, ~2% more per token above 4 (fitted:
// 1024x4096 .. 8192x28672 at 3-16 tokens).
double int4_mfma_us(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg) {
    mfma::Plan pl;
    if (!make_plan(M, K, G, batch, cfg, pl)) return 1e30;
    const uint32_t cu = cu_count();
    const double work = (double)pl.nsteps * pl.T * (pl.waves / 8.0) * ((pl.nwg + cu - 1) / cu);
    return 3.3 + 0.42 * work * (1.0 + 0.02 * ((double)batch - 4.0));
}

Int4Cfg int4_mfma_default(uint32_t, uint32_t, uint32_t) { return Int4Cfg{0, 0}; }

// Buffer loads address with 32-bit offsets: W, the scales and x must each
// span less than 2 GiB.
bool int4_mfma_supported(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg) {
    if (batch < 1 || batch > 16 || M == 0) return false;
    if (!(G == 32 || G == 64 || G == 128) || K % 128) return false;
    if ((uint64_t)M * K / 2 >= (1ull << 31)) return false;
    mfma::Plan pl;
    return make_plan(M, K, G, batch, cfg, pl);
}

hipError_t launch_int4_mfma(const uint32_t* W, const uint16_t* S, const uint16_t* B, int meta_kind,
                            bool interleaved, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                            uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg, hipStream_t s) {
    mfma::Plan pl;
    if (!make_plan(M, K, G, batch, cfg, pl)) return hipErrorInvalidValue;
    mfma::Args a;
    a.W = W;
    a.S = S;
    a.B = B;
    a.X = X;
    a.Y = Y;
    a.M = M;
    a.K = K;
    a.ntok = batch;
    a.y_f32 = y_f32 ? 1 : 0;
    a.gpr = K / G;
    a.P = pl.P;
    a.Q = pl.Q;
    a.J = pl.J;
    a.J8 = pl.J8;
    a.ngroups = ((M + mfma::kTile - 1) / mfma::kTile + pl.T - 1) / pl.T;
    a.groups_wg = pl.groups_wg;
    a.rounds = pl.rounds;
    a.nsteps = pl.nsteps;
    a.part_bytes = (uint32_t)mfma::lds_part(pl.waves, pl.T, pl.rounds, pl.P);
    const bool bf = meta_kind == 1;
    if (G == 32) return launch_mfma_g32(a, pl, interleaved, bf, s);
    if (G == 64) return launch_mfma_g64(a, pl, interleaved, bf, s);
    return launch_mfma_g128(a, pl, interleaved, bf, s);
}

}  // namespace kq
