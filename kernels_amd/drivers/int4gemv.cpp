// int4gemv -- host driver of the int4 group-affine GEMV (and its batched
// skinny-GEMM form) on libkq; mirrors int4-gemv/src/main.mm:120-572.
//
//   int4gemv [--M 4096] [--K 14336] [--G 64] [--batch 1] [--y f16|f32]
//            [--dist cfg|ref] [--rot-mb 1024] [--iters 50] [--warmup 10]
//            [--repeat 0] [--dump DIR]
//
// --dist cfg: the benchmark configuration (scale |N(0,0.02)|, bias
// N(0,0.02), x N(0,1)); --dist ref: the reference driver's distributions
// (scale U(-1,1)*0.02, bias U(-1,1)*0.15, x U(-1,1), int4-gemv/src/main.mm:
// 187-207). Both draw from mt19937(12345) in the reference's order.
#include <random>

#include "common.h"

int main(int argc, char** argv) {
    const drv::Args args(argc, argv);
    if (args.flag("--help")) {
        printf("int4gemv [--M m] [--K k] [--G g] [--batch b] [--y f16|f32] [--dist cfg|ref]\n"
               "         [--rot-mb mb] [--iters n] [--warmup n] [--repeat n] [--dump dir]\n");
        return 0;
    }
    const uint32_t M = (uint32_t)args.num("--M", 4096), K = (uint32_t)args.num("--K", 14336);
    const uint32_t G = (uint32_t)args.num("--G", 64), batch = (uint32_t)args.num("--batch", 1);
    const bool yf32 = args.str("--y", "f16") == "f32";
    const bool refdist = args.str("--dist", "cfg") == "ref";
    const size_t rot = (size_t)args.num("--rot-mb", 1024) << 20;
    const int iters = (int)args.num("--iters", 50), warmup = (int)args.num("--warmup", 10);
    int repeat = (int)args.num("--repeat", 0);
    const std::string dump = args.str("--dump", "");
    if (K % 32 || !(G == 32 || G == 64 || G == 128) || K % G || batch < 1 || batch > 16 || M == 0)
        drv::die("need K % 32 == 0, G in {32, 64, 128}, K % G == 0, 1 <= batch <= 16");

    printf("%s\nint4 GEMV  M=%u K=%u G=%u batch=%u  y=%s  dist=%s\n", kq_version(), M, K, G, batch,
           yf32 ? "f32" : "f16", refdist ? "ref" : "cfg");

    // ---- buffers (one generated set, copied NCOPY times on the device)
    const size_t wwords = (size_t)M * (K / 8), ngr = (size_t)M * (K / G);
    const size_t wbytes = wwords * 4, sbytes = ngr * 2;
    const size_t set_bytes = wbytes + 4 * sbytes;  // W + S + B + SB (all layouts kept)
    const uint32_t ncopy = drv::n_copies(set_bytes, rot);
    std::vector<uint32_t> W(wwords);
    std::vector<uint16_t> S(ngr), B(ngr), SB(2 * ngr), X((size_t)batch * K);
    std::mt19937 rng(12345);
    std::uniform_int_distribution<uint32_t> ud;
    std::uniform_real_distribution<float> uf(-1.0f, 1.0f);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    for (auto& w : W) w = ud(rng);
    for (size_t i = 0; i < ngr; ++i) {
        if (refdist) {
            S[i] = drv::f2h(uf(rng) * 0.02f);
            B[i] = drv::f2h(uf(rng) * 0.15f);
        } else {
            S[i] = drv::f2h(std::fabs(nd(rng)) * 0.02f);
            B[i] = drv::f2h(nd(rng) * 0.02f);
        }
        SB[2 * i] = S[i];
        SB[2 * i + 1] = B[i];
    }
    for (auto& x : X) x = drv::f2h(refdist ? uf(rng) : nd(rng));

    drv::DevBuf<uint32_t> dW(wwords * ncopy);
    drv::DevBuf<uint16_t> dS(ngr * ncopy), dB(ngr * ncopy), dSB(2 * ngr * ncopy);
    for (uint32_t c = 0; c < ncopy; ++c) {
        dW.upload(W.data(), wwords, c * wwords);
        dS.upload(S.data(), ngr, c * ngr);
        dB.upload(B.data(), ngr, c * ngr);
        dSB.upload(SB.data(), 2 * ngr, c * 2 * ngr);
    }
    drv::DevBuf<uint16_t> dX((size_t)batch * K);
    dX.upload(X.data(), X.size());
    const size_t ysz = yf32 ? 4 : 2, ycount = (size_t)batch * M;
    drv::DevBuf<uint8_t> dY(ycount * ysz);
    drv::DevBuf<uint32_t> sink(4);
    printf("weight copies rotated : %u x %.1f MB = %.0f MB distinct\n", ncopy, set_bytes / 1048576.0,
           ncopy * set_bytes / 1048576.0);

    hipStream_t st;
    DRV_HIP(hipStreamCreate(&st));
    const kq_stream_t ks = reinterpret_cast<kq_stream_t>(st);
    const kq_dtype yd = yf32 ? KQ_F32 : KQ_F16;
    const double bytes_call = (double)wbytes + 2.0 * sbytes + 2.0 * batch * K + (double)ysz * batch * M;
    uint32_t copy = 0;
    auto next_copy = [&]() { return copy = (copy + 1) % ncopy; };

    std::vector<drv::Variant> vars;
    auto add = [&](const char* name, kq_int4_path path, bool interleaved) {
        // refuse variants the library cannot run for this shape (checked once)
        const kq_status probe =
            interleaved ? kq_int4_gemv_path(dW.p, dSB.p, nullptr, KQ_F16, dX.p, dY.p, yd, M, K, G,
                                            batch, path, ks)
                        : kq_int4_gemv_path(dW.p, dS.p, dB.p, KQ_F16, dX.p, dY.p, yd, M, K, G,
                                            batch, path, ks);
        if (probe == KQ_EUNSUPPORTED) {
            printf("  (%s: not supported for this shape)\n", name);
            return;
        }
        DRV_KQ(probe);
        drv::Variant v;
        v.name = name;
        v.bytes = bytes_call;
        v.enc = [&, path, interleaved](hipStream_t, int) {
            const uint32_t c = next_copy();
            if (interleaved)
                DRV_KQ(kq_int4_gemv_path(dW.p + c * wwords, dSB.p + c * 2 * ngr, nullptr, KQ_F16,
                                         dX.p, dY.p, yd, M, K, G, batch, path, ks));
            else
                DRV_KQ(kq_int4_gemv_path(dW.p + c * wwords, dS.p + c * ngr, dB.p + c * ngr, KQ_F16,
                                         dX.p, dY.p, yd, M, K, G, batch, path, ks));
        };
        vars.push_back(v);
    };
    add("auto, interleaved (scale, bias)", KQ_PATH_AUTO, true);
    add("auto, separate S, B", KQ_PATH_AUTO, false);
    add("vector path (dot2)", KQ_PATH_VALU, true);
    add("matrix-core path (mfma 16x16x32)", KQ_PATH_MFMA, true);
    {  // the streaming-read ceiling over the same rotation (int4-gemv/src/main.mm:419-438)
        drv::Variant v;
        v.name = "pure read (kq_stream_read)";
        v.bytes = (double)(wbytes / 16 * 16);
        v.check = false;
        v.enc = [&](hipStream_t, int) {
            DRV_KQ(kq_stream_read(dW.p + next_copy() * wwords, wbytes / 16 * 16, sink.p, ks));
        };
        vars.push_back(v);
    }
    if (repeat <= 0) repeat = drv::probe_repeat(vars[0], st);
    printf("dispatches per span   : %d\n", repeat);

    // ---- fp64 host evaluation of Y on copy 0 (int4-gemv/src/main.mm:64-92)
    printf("computing the fp64 host check (%u x %u x %u) ...\n", M, K, batch);
    std::vector<double> yref(ycount);
    drv::par(M, [&](size_t m0, size_t m1) {
        std::vector<double> w(K);
        for (size_t m = m0; m < m1; ++m) {
            for (uint32_t k = 0; k < K; ++k) {
                const uint32_t q = (W[m * (K / 8) + k / 8] >> (4 * (k % 8))) & 0xF;
                const size_t g = m * (K / G) + k / G;
                w[k] = (double)drv::h2f(S[g]) * q + (double)drv::h2f(B[g]);
            }
            for (uint32_t b = 0; b < batch; ++b) {
                double a = 0;
                for (uint32_t k = 0; k < K; ++k) a += w[k] * drv::h2f(X[(size_t)b * K + k]);
                yref[(size_t)b * M + m] = a;
            }
        }
    });

    // ---- every variant checked before anything is timed
    for (auto& v : vars) {
        if (!v.check) continue;
        dY.zero();
        copy = ncopy - 1;  // the next dispatch uses copy 0
        v.enc(st, 0);
        DRV_HIP(hipStreamSynchronize(st));
        const auto raw = dY.download(ycount * ysz);
        auto yat = [&](size_t i) -> double {
            if (yf32) return __builtin_bit_cast(float, *reinterpret_cast<const uint32_t*>(raw.data() + 4 * i));
            return drv::h2f(*reinterpret_cast<const uint16_t*>(raw.data() + 2 * i));
        };
        v.relerr = drv::rel_inf(ycount, yat, [&](size_t i) { return yref[i]; });
        if (v.relerr >= 2e-3) {
            printf("  %-38s MISMATCH  err/|ref|inf %.2e\n", v.name.c_str(), v.relerr);
            return 1;
        }
        if (!dump.empty()) {
            std::string fn = dump + "/y_";
            for (char c : v.name) fn += isalnum((unsigned char)c) ? c : '_';
            drv::write_file(fn + (yf32 ? ".f32" : ".f16"), raw.data(), raw.size());
        }
    }
    printf("all variants verified against the fp64 host check\n");

    drv::time_round_robin(vars, st, repeat, warmup, iters);
    const double ceil_gbs = vars.back().bytes / vars.back().best_s / 1e9;
    drv::print_table(vars, ceil_gbs);
    const drv::Variant* best = nullptr;
    for (const auto& v : vars)
        if (v.check && (!best || v.best_s < best->best_s)) best = &v;
    const double bg = best->bytes / best->best_s / 1e9;
    printf("\nbytes per GEMV        : %.2f MB\n", bytes_call / 1048576.0);
    printf("pure-read ceiling     : %.1f GB/s (%.1f%% of 8 TB/s)\n", ceil_gbs, 100.0 * ceil_gbs / drv::kPeakGBs);
    printf("best GEMV variant     : %s\n", best->name.c_str());
    printf("achieved bandwidth    : %.1f GB/s  (%.3f us per call)\n", bg, best->best_s * 1e6);
    printf("  %% of 8 TB/s peak    : %.1f%%\n", 100.0 * bg / drv::kPeakGBs);
    printf("  %% of stream ceiling : %.1f%%\n", 100.0 * bg / ceil_gbs);

    if (!dump.empty()) {  // copy 0 of the inputs (int4-gemv/src/main.mm:553-570)
        drv::write_file(dump + "/W.u32", W.data(), wbytes);
        drv::write_file(dump + "/S.f16", S.data(), sbytes);
        drv::write_file(dump + "/B.f16", B.data(), sbytes);
        drv::write_file(dump + "/x.f16", X.data(), X.size() * 2);
        FILE* f = fopen((dump + "/shape.txt").c_str(), "w");
        if (!f) drv::die("cannot write shape.txt");
        fprintf(f, "%u %u %u %u %s\n", M, K, G, batch, yf32 ? "f32" : "f16");
        fclose(f);
        printf("\ndumped tensors to %s\n", dump.c_str());
    }
    DRV_HIP(hipStreamDestroy(st));
    return 0;
}
