// vqgemv -- host driver of the codebook (VQ, d = 2, 256 entries) dequant-GEMV
// on libkq, timed against the int4 GEMV at equal bytes per parameter; mirrors
// vq-gemv/src/main.mm:92-473.
//
//   vqgemv [--M 16384] [--K 16384] [--format ref|cfg] [--batch 1]
//          [--rot-mb 1024] [--iters 15] [--warmup 5] [--repeat 0] [--dump DIR]
//
// --format ref: the reference's format and generators (one fp16 codebook per
// matrix ~ U(-1,1), an fp16 scale per 32 weights ~ U(-1,1)*0.05, x ~ U(-1,1);
// vq-gemv/src/main.mm:155-172). --format cfg: the benchmark configuration
// (a codebook per 256 rows ~ N(0,0.02), one scale per row |N(1,0.1)|, x ~
// N(0,1)). The int4 opponent (G = 64, interleaved fp16 scale/bias) has the
// same 0.5625 bytes per parameter as the reference format.
#include <random>

#include "common.h"

int main(int argc, char** argv) {
    const drv::Args args(argc, argv);
    if (args.flag("--help")) {
        printf("vqgemv [--M m] [--K k] [--format ref|cfg] [--batch b] [--rot-mb mb]\n"
               "       [--iters n] [--warmup n] [--repeat n] [--dump dir]\n");
        return 0;
    }
    const uint32_t M = (uint32_t)args.num("--M", 16384), K = (uint32_t)args.num("--K", 16384);
    const uint32_t batch = (uint32_t)args.num("--batch", 1), G = 64;
    const bool cfg = args.str("--format", "ref") == "cfg";
    const size_t rot = (size_t)args.num("--rot-mb", 1024) << 20;
    const int iters = (int)args.num("--iters", 15), warmup = (int)args.num("--warmup", 5);
    int repeat = (int)args.num("--repeat", 0);
    const std::string dump = args.str("--dump", "");
    if (K % 64 || M == 0 || batch < 1 || batch > 16) drv::die("need K % 64 == 0, M >= 1, 1 <= batch <= 16");

    const uint32_t rpc = cfg ? 256 : M, sg = cfg ? K : 32;
    const uint32_t ncb = (M + rpc - 1) / rpc;
    const size_t idx_bytes = (size_t)M * (K / 2), nscale = (size_t)M * (K / sg);
    const size_t wwords = (size_t)M * (K / 8), ngr = (size_t)M * (K / G);
    const size_t vq_set = idx_bytes + 2 * nscale, i4_set = wwords * 4 + 4 * ngr;
    const uint32_t ncopy = drv::n_copies(std::max(vq_set, i4_set), rot);

    printf("%s\nVQ GEMV  M=%u K=%u batch=%u  format=%s (codebook per %u rows, scale per %u)\n",
           kq_version(), M, K, batch, cfg ? "cfg" : "ref", rpc, sg);
    printf("VQ   d=2, 256 entries : %.4f bytes/param\n", (double)vq_set / ((double)M * K));
    printf("int4 affine g=%u      : %.4f bytes/param\n", G, (double)i4_set / ((double)M * K));
    printf("copies rotated        : %u (%.0f MB distinct per format)\n", ncopy,
           (double)std::max(vq_set, i4_set) * ncopy / 1048576.0);

    // ---- generators in the reference's order (vq-gemv/src/main.mm:155-172)
    std::mt19937 rng(12345);
    std::uniform_int_distribution<uint32_t> ud;
    std::uniform_real_distribution<float> uf(-1.0f, 1.0f);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::vector<uint8_t> IDX(idx_bytes);
    std::vector<uint16_t> C((size_t)ncb * 512), VS(nscale), SB(2 * ngr), X((size_t)batch * K);
    std::vector<uint32_t> W(wwords);
    for (auto& i : IDX) i = (uint8_t)(ud(rng) & 0xFF);
    for (auto& c : C) c = drv::f2h(cfg ? 0.02f * nd(rng) : uf(rng));
    for (auto& v : VS) v = drv::f2h(cfg ? std::fabs(1.0f + 0.1f * nd(rng)) : uf(rng) * 0.05f);
    for (auto& w : W) w = ud(rng);
    for (size_t i = 0; i < ngr; ++i) {
        SB[2 * i] = drv::f2h(uf(rng) * 0.02f);
        SB[2 * i + 1] = drv::f2h(uf(rng) * 0.15f);
    }
    for (auto& x : X) x = drv::f2h(cfg ? nd(rng) : uf(rng));

    drv::DevBuf<uint8_t> dIDX(idx_bytes * ncopy);
    drv::DevBuf<uint16_t> dVS(nscale * ncopy), dC(C.size()), dSB(2 * ngr * ncopy), dX(X.size());
    drv::DevBuf<uint32_t> dW(wwords * ncopy), sink(4);
    for (uint32_t c = 0; c < ncopy; ++c) {
        dIDX.upload(IDX.data(), idx_bytes, c * idx_bytes);
        dVS.upload(VS.data(), nscale, c * nscale);
        dW.upload(W.data(), wwords, c * wwords);
        dSB.upload(SB.data(), 2 * ngr, c * 2 * ngr);
    }
    dC.upload(C.data(), C.size());
    dX.upload(X.data(), X.size());
    const size_t ycount = (size_t)batch * M;
    drv::DevBuf<float> dY(ycount);

    hipStream_t st;
    DRV_HIP(hipStreamCreate(&st));
    const kq_stream_t ks = reinterpret_cast<kq_stream_t>(st);
    uint32_t copy = 0;
    auto next_copy = [&]() { return copy = (copy + 1) % ncopy; };

    // ---- fp64 host evaluations of both formats on copy 0 (vq-gemv/src/main.mm:51-80)
    printf("computing the fp64 host checks (%u rows x %u, both formats) ...\n", M, K);
    std::vector<double> yvq(ycount), yi4(ycount);
    drv::par(M, [&](size_t m0, size_t m1) {
        std::vector<double> w(K), u(K);
        for (size_t m = m0; m < m1; ++m) {
            const uint16_t* cb = C.data() + (m / rpc) * 512;
            for (uint32_t i = 0; i < K / 2; ++i) {
                const uint32_t c = IDX[m * (K / 2) + i];
                const double s = drv::h2f(VS[m * (K / sg) + 2 * i / sg]);
                w[2 * i] = s * drv::h2f(cb[2 * c]);
                w[2 * i + 1] = s * drv::h2f(cb[2 * c + 1]);
            }
            for (uint32_t k = 0; k < K; ++k) {
                const uint32_t q = (W[m * (K / 8) + k / 8] >> (4 * (k % 8))) & 0xF;
                const size_t g = m * (K / G) + k / G;
                u[k] = (double)drv::h2f(SB[2 * g]) * q + (double)drv::h2f(SB[2 * g + 1]);
            }
            for (uint32_t b = 0; b < batch; ++b) {
                double a = 0, a4 = 0;
                for (uint32_t k = 0; k < K; ++k) {
                    const double x = drv::h2f(X[(size_t)b * K + k]);
                    a += w[k] * x;
                    a4 += u[k] * x;
                }
                yvq[(size_t)b * M + m] = a;
                yi4[(size_t)b * M + m] = a4;
            }
        }
    });

    const double xy = 2.0 * batch * K + 4.0 * batch * M;
    std::vector<drv::Variant> vars(3);
    std::vector<const std::vector<double>*> refs = {&yvq, &yi4, nullptr};
    vars[0].name = "VQ (kq_vq_gemv)";
    vars[0].bytes = (double)vq_set + 1024.0 * ncb + xy;
    vars[0].enc = [&](hipStream_t, int) {
        const uint32_t c = next_copy();
        DRV_KQ(kq_vq_gemv(dIDX.p + c * idx_bytes, dC.p, dVS.p + c * nscale, dX.p, dY.p, KQ_F32, M,
                          K, rpc, sg, batch, ks));
    };
    vars[1].name = "int4 g64 at equal bytes";
    vars[1].bytes = (double)i4_set + xy;
    vars[1].enc = [&](hipStream_t, int) {
        const uint32_t c = next_copy();
        DRV_KQ(kq_int4_gemv(dW.p + c * wwords, dSB.p + c * 2 * ngr, nullptr, KQ_F16, dX.p, dY.p,
                            KQ_F32, M, K, G, batch, ks));
    };
    vars[2].name = "pure read (kq_stream_read)";
    vars[2].bytes = (double)(idx_bytes / 16 * 16);
    vars[2].check = false;
    vars[2].enc = [&](hipStream_t, int) {
        DRV_KQ(kq_stream_read(dIDX.p + next_copy() * idx_bytes, idx_bytes / 16 * 16, sink.p, ks));
    };

    for (size_t i = 0; i < vars.size(); ++i) {
        auto& v = vars[i];
        if (!v.check) continue;
        dY.zero();
        copy = ncopy - 1;
        v.enc(st, 0);
        DRV_HIP(hipStreamSynchronize(st));
        const auto y = dY.download(ycount);
        const auto& r = *refs[i];
        v.relerr = drv::rel_inf(ycount, [&](size_t j) { return (double)y[j]; }, [&](size_t j) { return r[j]; });
        if (v.relerr >= 2e-3) {
            printf("  %-38s MISMATCH  err/|ref|inf %.2e\n", v.name.c_str(), v.relerr);
            return 1;
        }
        if (!dump.empty()) {
            std::string fn = dump + "/y_";
            for (char c : v.name) fn += isalnum((unsigned char)c) ? c : '_';
            drv::write_file(fn + ".f32", y.data(), y.size() * 4);
        }
    }
    printf("all variants verified against their fp64 host check\n");
    if (repeat <= 0) repeat = drv::probe_repeat(vars[0], st);
    printf("dispatches per span   : %d\n", repeat);

    drv::time_round_robin(vars, st, repeat, warmup, iters);
    const double ceil_gbs = vars[2].bytes / vars[2].best_s / 1e9;
    drv::print_table(vars, ceil_gbs);
    const auto &vq = vars[0], &i4 = vars[1];
    const double gv = vq.bytes / vq.best_s / 1e9, gi = i4.bytes / i4.best_s / 1e9;
    printf("\nVQ                    : %.1f GB/s  (%.1f%% of peak, %.1f%% of ceiling)  %.3f us\n", gv,
           100.0 * gv / drv::kPeakGBs, 100.0 * gv / ceil_gbs, vq.best_s * 1e6);
    printf("int4 at equal bytes   : %.1f GB/s  (%.1f%% of peak)  %.3f us\n", gi,
           100.0 * gi / drv::kPeakGBs, i4.best_s * 1e6);
    printf("VQ / int4 throughput  : %.3fx\n", i4.best_s / vq.best_s);

    if (!dump.empty()) {
        drv::write_file(dump + "/IDX.u8", IDX.data(), IDX.size());
        drv::write_file(dump + "/C.f16", C.data(), C.size() * 2);
        drv::write_file(dump + "/S.f16", VS.data(), VS.size() * 2);
        drv::write_file(dump + "/W.u32", W.data(), W.size() * 4);
        drv::write_file(dump + "/SB.f16", SB.data(), SB.size() * 2);
        drv::write_file(dump + "/x.f16", X.data(), X.size() * 2);
        FILE* f = fopen((dump + "/shape.txt").c_str(), "w");
        if (!f) drv::die("cannot write shape.txt");
        fprintf(f, "%u %u %u %u %u\n", M, K, rpc, sg, batch);
        fclose(f);
        printf("\ndumped tensors to %s\n", dump.c_str());
    }
    DRV_HIP(hipStreamDestroy(st));
    return 0;
}
