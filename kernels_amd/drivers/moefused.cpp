// moefused -- host driver of the gpt-oss-120b MoE decode block on libkq;
// mirrors moe-fused/src/main.mm:74-428.
//
//   moefused [--store experts.bin] [--experts 128] [--batch 1] [--resident 8]
//            [--iters 30] [--warmup 8] [--repeat 20] [--layers 36]
//            [--router f32|f16] [--dump DIR]
//
// The expert pool is the reference's on-disk blob layout (14,024,704 B per
// expert, moe-fused/src/main.mm:23-25): read from --store with pread, as the
// reference does (moe-fused/src/main.mm:129-149), or generated (uniform
// nibbles; bf16 scale |N(0.0064, 0.001)|, bias N(-0.048, 0.004), output bias
// N(0, 0.02): the statistics of int4-quantised N(0, 0.02) weights). Router
// weights and the token are the reference's closed-form LCG
// (moe-fused/src/main.mm:160-171); token b > 0 shifts the x pattern by 7b.
//
// --resident copies of the pool are kept in HBM and the blocks of a span
// cycle through them, so a block never finds its experts in the 256 MB MALL
// from the block before (the same experts at distinct addresses, like the
// layers of a decode step).
#include <fcntl.h>
#include <unistd.h>

#include <random>

#include "common.h"

namespace {

// fp64 host evaluation of one projection row range of one expert blob
// (moe-fused/src/main.mm:45-62): bf16 scale/bias per 64, bf16 output bias.
void proj_f64(const uint8_t* blob, const kq_moe_desc& d, uint64_t off, const double* x, double* y,
              uint32_t K, size_t m0, size_t m1) {
    const uint32_t* W = reinterpret_cast<const uint32_t*>(blob + off + d.sub_w);
    const uint16_t* S = reinterpret_cast<const uint16_t*>(blob + off + d.sub_s);
    const uint16_t* B = reinterpret_cast<const uint16_t*>(blob + off + d.sub_b);
    const uint16_t* BI = reinterpret_cast<const uint16_t*>(blob + off + d.sub_bi);
    for (size_t m = m0; m < m1; ++m) {
        double a = 0;
        for (uint32_t k = 0; k < K; ++k) {
            const uint32_t q = (W[m * (K / 8) + k / 8] >> (4 * (k % 8))) & 0xF;
            const size_t g = m * (K / 64) + k / 64;
            a += ((double)drv::bf2f(S[g]) * q + (double)drv::bf2f(B[g])) * x[k];
        }
        y[m] = a + (double)drv::bf2f(BI[m]);
    }
}

void fill_expert(uint8_t* blob, const kq_moe_desc& d, uint32_t seed) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    for (size_t i = 0; i + 4 <= d.blob; i += 4) {
        const uint32_t r = rng();
        memcpy(blob + i, &r, 4);
    }
    const uint64_t offs[3] = {d.off_gate, d.off_up, d.off_down};
    const uint32_t rows[3] = {d.inter, d.inter, d.hidden}, cols[3] = {d.hidden, d.hidden, d.inter};
    for (int p = 0; p < 3; ++p) {
        uint16_t* S = reinterpret_cast<uint16_t*>(blob + offs[p] + d.sub_s);
        uint16_t* B = reinterpret_cast<uint16_t*>(blob + offs[p] + d.sub_b);
        uint16_t* BI = reinterpret_cast<uint16_t*>(blob + offs[p] + d.sub_bi);
        const size_t ng = (size_t)rows[p] * (cols[p] / 64);
        for (size_t g = 0; g < ng; ++g) {
            S[g] = drv::f2bf(std::fabs(0.0064f + 0.001f * nd(rng)));
            B[g] = drv::f2bf(-0.048f + 0.004f * nd(rng));
        }
        for (uint32_t m = 0; m < rows[p]; ++m) BI[m] = drv::f2bf(0.02f * nd(rng));
    }
}

}  // namespace

int main(int argc, char** argv) {
    const drv::Args args(argc, argv);
    if (args.flag("--help")) {
        printf("moefused [--store experts.bin] [--experts n] [--batch b] [--resident n]\n"
               "         [--iters n] [--warmup n] [--repeat n] [--layers n] [--router f32|f16]\n"
               "         [--dump dir]\n");
        return 0;
    }
    kq_moe_desc d;
    kq_moe_default_desc(&d);
    d.n_experts = (uint32_t)args.num("--experts", d.n_experts);
    const uint32_t batch = (uint32_t)args.num("--batch", 1);
    const uint32_t nres = (uint32_t)std::max(1L, args.num("--resident", 8));
    const int iters = (int)args.num("--iters", 30), warmup = (int)args.num("--warmup", 8);
    const int repeat = (int)args.num("--repeat", 20), layers = (int)args.num("--layers", 36);
    const bool rf16 = args.str("--router", "f32") == "f16";
    const std::string store = args.str("--store", ""), dump = args.str("--dump", "");
    if (batch < 1 || batch > 16 || d.n_experts < d.top_k) drv::die("need 1 <= batch <= 16, experts >= top_k");
    const uint32_t HID = d.hidden, INTER = d.inter, NE = d.n_experts, TK = d.top_k;

    printf("%s\n", kq_version());
    printf("block                 : hidden=%u inter=%u  %u experts, top-%u, batch %u  (gpt-oss-120b, int4 g=64)\n",
           HID, INTER, NE, TK, batch);
    const size_t pool_bytes = (size_t)NE * d.blob;
    printf("resident experts      : %.2f GB x %u copies\n", pool_bytes / 1e9, nres);

    // ---- the expert pool
    std::vector<uint8_t> pool(pool_bytes);
    const auto t0 = std::chrono::steady_clock::now();
    if (!store.empty()) {
        const int fd = open(store.c_str(), O_RDONLY);
        if (fd < 0) drv::die("cannot open " + store);
        printf("loading %u experts from %s ...", NE, store.c_str());
        fflush(stdout);
        for (size_t got = 0; got < pool_bytes;) {
            const ssize_t n = pread(fd, pool.data() + got, pool_bytes - got, (off_t)got);
            if (n <= 0) drv::die("pread " + store);
            got += (size_t)n;
        }
        close(fd);
    } else {
        printf("generating %u experts ...", NE);
        fflush(stdout);
        drv::par(NE, [&](size_t e0, size_t e1) {
            for (size_t e = e0; e < e1; ++e) fill_expert(pool.data() + e * d.blob, d, 12345u + (uint32_t)e);
        });
    }
    printf(" %.1f s\n", std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
    std::vector<drv::DevBuf<uint8_t>*> dpool;
    for (uint32_t c = 0; c < nres; ++c) {
        dpool.push_back(new drv::DevBuf<uint8_t>(pool_bytes));
        if (c == 0)
            dpool[0]->upload(pool.data(), pool_bytes);
        else
            DRV_HIP(hipMemcpy(dpool[c]->p, dpool[0]->p, pool_bytes, hipMemcpyDeviceToDevice));
    }

    // ---- router and tokens (moe-fused/src/main.mm:160-171)
    std::vector<float> R((size_t)NE * HID), X((size_t)batch * HID);
    for (size_t i = 0; i < R.size(); ++i) {
        const uint32_t h = (uint32_t)(i * 1103515245u + 12345u) >> 16;
        R[i] = 0.02f * ((int)(h % 2001) - 1000) / 1000.0f;
    }
    for (uint32_t b = 0; b < batch; ++b)
        for (uint32_t i = 0; i < HID; ++i) X[(size_t)b * HID + i] = 0.05f * ((int)((i + 7 * b) % 17) - 8);
    std::vector<uint16_t> Rh(R.size());
    for (size_t i = 0; i < R.size(); ++i) Rh[i] = drv::f2h(R[i]);
    drv::DevBuf<float> dR(R.size()), dX(X.size()), dWgt((size_t)batch * TK), dY((size_t)batch * HID);
    drv::DevBuf<uint16_t> dRh(R.size()), dXh((size_t)batch * HID), dH((size_t)batch * TK * INTER);
    drv::DevBuf<uint32_t> dIdx((size_t)batch * TK);
    dR.upload(R.data(), R.size());
    dRh.upload(Rh.data(), Rh.size());
    dX.upload(X.data(), X.size());
    const void* rptr = rf16 ? static_cast<const void*>(dRh.p) : static_cast<const void*>(dR.p);
    const kq_dtype rdt = rf16 ? KQ_F16 : KQ_F32;
    const size_t wsb = kq_moe_workspace_size(&d, batch);
    if (wsb == 0) drv::die("kq_moe_workspace_size");
    drv::DevBuf<uint8_t> ws(wsb);

    hipStream_t st;
    DRV_HIP(hipStreamCreate(&st));
    const kq_stream_t ks = reinterpret_cast<kq_stream_t>(st);
    DRV_KQ(kq_moe_workspace_init(ws.p, wsb, ks));

    // ---- fp64 host evaluation (moe-fused/src/main.mm:300-334)
    printf("computing the fp64 host check ...\n");
    std::vector<uint32_t> ridx((size_t)batch * TK);
    std::vector<double> rwgt((size_t)batch * TK), yref((size_t)batch * HID, 0.0);
    for (uint32_t b = 0; b < batch; ++b) {
        std::vector<double> xd(HID), lg(NE);
        for (uint32_t i = 0; i < HID; ++i) xd[i] = X[(size_t)b * HID + i];
        for (uint32_t e = 0; e < NE; ++e) {
            double s = 0;
            for (uint32_t k = 0; k < HID; ++k)
                s += (rf16 ? (double)drv::h2f(Rh[(size_t)e * HID + k]) : (double)R[(size_t)e * HID + k]) * xd[k];
            lg[e] = s;
        }
        std::vector<double> sel(TK);
        for (uint32_t j = 0; j < TK; ++j) {  // strict >, ascending scan: lowest index wins ties
            uint32_t bi = 0;
            double bv = -1e300;
            for (uint32_t e = 0; e < NE; ++e)
                if (lg[e] > bv) bv = lg[e], bi = e;
            ridx[(size_t)b * TK + j] = bi;
            sel[j] = bv;
            lg[bi] = -1e300;
        }
        double sm = 0;
        for (uint32_t j = 0; j < TK; ++j) sm += rwgt[(size_t)b * TK + j] = std::exp(sel[j] - sel[0]);
        for (uint32_t j = 0; j < TK; ++j) rwgt[(size_t)b * TK + j] /= sm;
        // the projections see fp16(x), as the kernels do
        for (auto& v : xd) v = drv::h2f(drv::f2h((float)v));
        for (uint32_t j = 0; j < TK; ++j) {
            const uint8_t* blob = pool.data() + (size_t)ridx[(size_t)b * TK + j] * d.blob;
            std::vector<double> g(INTER), u(INTER), h(INTER), yy(HID);
            drv::par(INTER, [&](size_t a, size_t c) { proj_f64(blob, d, d.off_gate, xd.data(), g.data(), HID, a, c); });
            drv::par(INTER, [&](size_t a, size_t c) { proj_f64(blob, d, d.off_up, xd.data(), u.data(), HID, a, c); });
            for (uint32_t i = 0; i < INTER; ++i) {
                const double gg = std::min(g[i], 7.0), ll = std::max(-7.0, std::min(u[i], 7.0));
                h[i] = drv::h2f(drv::f2h((float)((gg / (1.0 + std::exp(-1.702 * gg))) * (ll + 1.0))));
            }
            drv::par(HID, [&](size_t a, size_t c) { proj_f64(blob, d, d.off_down, h.data(), yy.data(), INTER, a, c); });
            for (uint32_t i = 0; i < HID; ++i) yref[(size_t)b * HID + i] += rwgt[(size_t)b * TK + j] * yy[i];
        }
    }

    // ---- variants: the block in one call, and the three passes as three calls
    int layer = 0;
    auto fused = [&](hipStream_t, int) {
        DRV_KQ(kq_moe_block(dpool[layer]->p, &d, rptr, rdt, dX.p, KQ_F32, batch, dIdx.p, dWgt.p, dXh.p,
                            dH.p, dY.p, KQ_F32, ws.p, wsb, ks));
        layer = (layer + 1) % (int)nres;
    };
    auto three = [&](hipStream_t, int) {
        DRV_KQ(kq_moe_router_topk(rptr, rdt, dX.p, KQ_F32, batch, &d, dIdx.p, dWgt.p, dXh.p, ws.p, wsb, ks));
        DRV_KQ(kq_moe_gate_up_swiglu(dpool[layer]->p, &d, dIdx.p, dXh.p, dH.p, batch, nullptr, 0, ks));
        DRV_KQ(kq_moe_down_combine(dpool[layer]->p, &d, dIdx.p, dWgt.p, dH.p, dY.p, KQ_F32, batch, nullptr, 0, ks));
        layer = (layer + 1) % (int)nres;
    };
    // one operation per launch (encodeUnfused, moe-fused/src/main.mm:208-284); one token only
    const size_t uwsb = kq_moe_unfused_workspace_size(&d);
    drv::DevBuf<uint8_t> uws(uwsb ? uwsb : 256);
    uint32_t nunf = 0;
    auto unfused = [&](hipStream_t, int) {
        DRV_KQ(kq_moe_block_unfused(dpool[layer]->p, &d, rptr, rdt, dX.p, KQ_F32, batch, dIdx.p, dWgt.p,
                                    dXh.p, dH.p, dY.p, KQ_F32, uws.p, uwsb, &nunf, ks));
        layer = (layer + 1) % (int)nres;
    };
    std::vector<drv::Variant> vars(2);
    vars[0].name = "fused block (kq_moe_block)";
    vars[0].enc = fused;
    vars[0].launches = 3;
    vars[1].name = "router, gate_up, down (3 calls)";
    vars[1].enc = three;
    vars[1].launches = 3;
    if (batch == 1) {
        vars.emplace_back();
        vars[2].name = "unfused (one op per launch)";
        vars[2].enc = unfused;
        vars[2].launches = 3 + 5 * (int)TK;
    }

    printf("\ncorrectness vs the fp64 host check (router, top-k, both matmuls, SwiGLU)\n");
    double yinf = 0;
    for (double v : yref) yinf = std::max(yinf, std::fabs(v));
    bool ok = true;
    std::vector<float> y;
    std::vector<uint32_t> gi;
    std::vector<float> gw;
    for (auto& v : vars) {
        dY.zero();
        layer = 0;
        v.enc(st, 0);
        DRV_HIP(hipStreamSynchronize(st));
        y = dY.download(dY.n);
        gi = dIdx.download(dIdx.n);
        gw = dWgt.download(dWgt.n);
        const bool idxok = gi == ridx;
        if (!idxok) {
            printf("      gpu idx/wgt:");
            for (size_t j = 0; j < gi.size(); ++j) printf(" %u:%.6f", gi[j], gw[j]);
            printf("\n      ref idx/wgt:");
            for (size_t j = 0; j < ridx.size(); ++j) printf(" %u:%.6f", ridx[j], rwgt[j]);
            printf("\n");
        }
        double e = 0;
        for (size_t i = 0; i < y.size(); ++i) e = std::max(e, std::fabs((double)y[i] - yref[i]));
        v.relerr = e / std::max(yinf, 1e-30);
        printf("  %-34s top-k %s   max|d|/|y|inf = %.2e  %s\n", v.name.c_str(), idxok ? "match" : "MISMATCH",
               v.relerr, (idxok && v.relerr < 2e-3) ? "ok" : "FAIL");
        ok = ok && idxok && v.relerr < 2e-3;
    }
    if (batch == 1 && nunf != (uint32_t)vars[2].launches) {
        printf("unfused path reported %u launches, expected %d\n", nunf, vars[2].launches);
        return 1;
    }
    if (!ok) return 1;
    if (!dump.empty()) {  // results/topk.txt and results/y_metal.f32 of the reference
        FILE* f = fopen((dump + "/topk.txt").c_str(), "w");
        if (!f) drv::die("cannot write topk.txt");
        for (size_t j = 0; j < gi.size(); ++j) fprintf(f, "%u %.9f\n", gi[j], gw[j]);
        fclose(f);
        drv::write_file(dump + "/y.f32", y.data(), y.size() * 4);
        for (size_t j = 0; j < gi.size(); ++j) {
            const std::string fn = dump + "/expert_" + std::to_string(gi[j]) + ".bin";
            drv::write_file(fn, pool.data() + (size_t)gi[j] * d.blob, d.blob);
        }
        printf("dumped topk.txt, y.f32 and the selected experts to %s\n", dump.c_str());
    }

    // ---- timing: best over iters of spans of `repeat` blocks (moe-fused/src/main.mm:378-392)
    drv::time_round_robin(vars, st, repeat, warmup, iters);
    std::vector<uint32_t> uniq(gi);
    std::sort(uniq.begin(), uniq.end());
    uniq.erase(std::unique(uniq.begin(), uniq.end()), uniq.end());
    const double per_exp = 3.0 * ((double)INTER * HID / 2 + 4.0 * INTER * (HID / 64) + 2.0 * INTER);
    const double router = (double)NE * HID * (rf16 ? 2 : 4);
    const double bytes = uniq.size() * per_exp + router;
    const double ref_mb = TK * 3.0 * 4147200 + TK * 6.0 * 259200;  // moe-fused/src/main.mm:408
    for (auto& v : vars) v.bytes = bytes;
    printf("\nbytes read per block  : %.2f MB (%zu distinct experts x 3 projections + router)\n", bytes / 1e6,
           uniq.size());
    printf("\n%-36s %10s %12s %12s %12s %12s\n", "path", "launches", "us/block", "GB/s", "GB/s(ref)", "tok/s");
    printf("------------------------------------------------------------------------------------------------\n");
    for (const auto& v : vars)
        printf("  %-34s %10d %12.3f %12.1f %12.1f %12.1f\n", v.name.c_str(), v.launches, v.best_s * 1e6,
               bytes / v.best_s / 1e9, ref_mb / v.best_s / 1e9, batch / (layers * v.best_s));
    printf("------------------------------------------------------------------------------------------------\n");
    const double tb = std::min(vars[0].best_s, vars[1].best_s);
    printf("\nblock time            : %.3f us (median %.3f us)\n", tb * 1e6, vars[0].med_s * 1e6);
    printf("%% of 8 TB/s on bytes read : %.1f%%\n", 100.0 * bytes / tb / 1e9 / drv::kPeakGBs);
    if (batch == 1)
        printf("unfused / fused       : %.2fx the time, %d vs %d launches (%.2f us per extra launch)\n",
               vars[2].best_s / vars[0].best_s, vars[2].launches, vars[0].launches,
               (vars[2].best_s - vars[0].best_s) * 1e6 / (vars[2].launches - vars[0].launches));
    printf("decode rate           : %.1f tok/s  (%d layers, experts resident, MoE only)\n",
           batch / (layers * tb), layers);

    DRV_HIP(hipStreamDestroy(st));
    for (auto* p : dpool) delete p;
    return 0;
}
