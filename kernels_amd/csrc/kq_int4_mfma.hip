// kq_int4_mfma.hip -- launch planning for the matrix-core int4 path (the
// kernel is in kq_int4_mfma_kernel.h, instantiated per quant-group size in
// kq_int4_mfma_g{32,64,128}.hip).
//
// A plan fixes the split of the 16 waves of a workgroup into P K-parts and
// Q tile lanes (P divides the number of 128-k spans), the tiles per
// workgroup (at most one workgroup per CU: ceil(tiles / CUs) tiles, in
// rounds of Q), and the ring depth D. Among the P that fit the LDS, the plan
// with the least per-workgroup work (waves x padded steps) wins; fewer than
// 8 waves count as proportionally slower (too little in flight).
#include "kq_int4_mfma_kernel.h"

namespace kq {

namespace {

int g_ncu = 0;
uint32_t ncu() {
    if (g_ncu <= 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            n > 0)
            g_ncu = n;
        else
            g_ncu = 256;
    }
    return (uint32_t)g_ncu;
}

constexpr size_t kLdsMax = 160 * 1024;

bool make_plan(uint32_t M, uint32_t K, uint32_t G, uint32_t ntok, Int4Cfg cfg, mfma::Plan& out) {
    const uint32_t nspan = K / 128, ntiles = (M + mfma::kTile - 1) / mfma::kTile, cu = ncu();
    const uint32_t rmax = ntok == 1 ? 1 : 4;
    if (cfg.unroll != 0 && cfg.unroll != 2 && cfg.unroll != 4 && cfg.unroll != 8) return false;
    bool found = false;
    double best = 0.0;
    for (uint32_t P = mfma::kMaxWaves; P >= 1; --P) {
        if (nspan % P) continue;
        if (cfg.rows > 0 && (uint32_t)cfg.rows != P) continue;
        const uint32_t Q = mfma::kMaxWaves / P, waves = P * Q, J = nspan / P;
        const uint32_t per_cu = (ntiles + cu - 1) / cu;
        const uint32_t rounds = (per_cu + Q - 1) / Q;
        const uint32_t tiles_wg = rounds * Q;
        const uint32_t nwg = (ntiles + tiles_wg - 1) / tiles_wg;
        const uint32_t nreal = rounds * J;
        const uint32_t D = cfg.unroll > 0 ? (uint32_t)cfg.unroll : nreal >= 8 ? 8 : nreal >= 4 ? 4 : 2;
        const uint32_t nsteps = (nreal + D - 1) / D * D;
        const size_t lds = mfma::lds_xp(ntok, K) + mfma::lds_xk(ntok, K, G) + mfma::lds_part(waves, rmax);
        if (lds > kLdsMax) continue;
        const double cost = (double)nsteps * waves * (waves < 8 ? 8.0 / waves : 1.0);
        if (!found || cost < best) {
            found = true;
            best = cost;
            out = mfma::Plan{P, Q, J, rounds, tiles_wg, nwg, nreal, nsteps, D, rmax, lds};
        }
    }
    return found;
}

// Most tokens (<= 16) one pass can stage.
uint32_t tokens_per_pass(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg) {
    mfma::Plan pl;
    for (uint32_t t = batch < 16 ? batch : 16; t >= 1; --t)
        if (make_plan(M, K, G, t, cfg, pl)) return t;
    return 0;
}

}  // namespace

uint32_t int4_mfma_tokens_per_pass(uint32_t M, uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg) {
    return tokens_per_pass(M, K, G, batch, cfg);
}

Int4Cfg int4_mfma_default(uint32_t, uint32_t, uint32_t) { return Int4Cfg{0, 0}; }

bool int4_mfma_supported(uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg) {
    if (batch < 1 || batch > 16) return false;
    if (!(G == 32 || G == 64 || G == 128) || K % 128) return false;
    return tokens_per_pass(16, K, G, 1, cfg) >= 1;
}

hipError_t launch_int4_mfma(const uint32_t* W, const uint16_t* S, const uint16_t* B, int meta_kind,
                            bool interleaved, const uint16_t* X, void* Y, bool y_f32, uint32_t M,
                            uint32_t K, uint32_t G, uint32_t batch, Int4Cfg cfg, hipStream_t s) {
    const uint32_t per_pass = tokens_per_pass(M, K, G, batch, cfg);
    if (per_pass == 0) return hipErrorInvalidValue;
    const size_t ysz = y_f32 ? 4 : 2;
    for (uint32_t t0 = 0; t0 < batch;) {
        const uint32_t nt = batch - t0 < per_pass ? batch - t0 : per_pass;
        mfma::Plan pl;
        if (!make_plan(M, K, G, nt, cfg, pl)) return hipErrorInvalidValue;
        mfma::Args a;
        a.W = W;
        a.S = S;
        a.B = B;
        a.X = X + (size_t)t0 * K;
        a.Y = reinterpret_cast<uint8_t*>(Y) + (size_t)t0 * M * ysz;
        a.M = M;
        a.K = K;
        a.ntok = nt;
        a.y_f32 = y_f32 ? 1 : 0;
        a.nspan = K / 128;
        a.gpr = K / G;
        a.P = pl.P;
        a.Q = pl.Q;
        a.J = pl.J;
        a.tiles_wg = pl.tiles_wg;
        a.ntiles = (M + mfma::kTile - 1) / mfma::kTile;
        a.rounds = pl.rounds;
        a.nreal = pl.nreal;
        a.nsteps = pl.nsteps;
        const bool bf = meta_kind == 1;
        hipError_t e;
        if (G == 32) e = launch_mfma_g32(a, pl, interleaved, bf, s);
        else if (G == 64) e = launch_mfma_g64(a, pl, interleaved, bf, s);
        else e = launch_mfma_g128(a, pl, interleaved, bf, s);
        if (e != hipSuccess) return e;
        t0 += nt;
    }
    return hipSuccess;
}

}  // namespace kq
