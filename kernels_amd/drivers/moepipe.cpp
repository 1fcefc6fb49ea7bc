// moepipe -- expert streaming from a store file into HBM, with each expert's
// gate/up + SwiGLU and down computed by libkq as it arrives; mirrors
// moe-pipeline/src/main.mm (its seq / io / pipe drivers and report).
//
//   moepipe --store experts.bin [--experts 288] [--depth 3] [--workers 4]
//           [--reps 3] [--mode all|seq|io|pipe] [--hbm-slots 2] [--warm]
//           [--verify DIR]
//
// The store is the on-disk blob layout of gpt-oss-120b experts (14,024,704 B
// each, moe-fused/src/main.mm:23-25), any number of them. Run i reads store
// expert (i * 2654435761) mod n_store, a bijection on the store (2654435761 is
// prime), so no expert is read twice while --experts <= n_store.
//
// Path of one expert: a reader thread preads it (O_DIRECT when the kernel
// takes it for pinned pages; otherwise the store is evicted from the page
// cache before every run unless --warm) into a pinned host slot; hipMemcpyAsync on a copy stream
// moves it into one of --hbm-slots HBM slots once the compute that last used
// that slot is done (event); the compute stream waits for the copy (event)
// and runs kq_moe_gate_up_swiglu + kq_moe_down_combine on the slot as a
// one-expert pool (n_experts = top_k = 1, weight 1), writing that expert's y
// into a per-run result array. The host never waits for the GPU inside the
// loop, only for reads.
//
//   seq  : read expert i on the calling thread, copy, compute, wait; then i+1.
//   io   : reads only (the ceiling the pipeline chases).
//   pipe : depth reads in flight; at step i wait for read i, submit read
//          i + depth (refill before compute, moe-pipeline/src/main.mm:348-357)
//          into host slot (i + depth) % (depth + 2) once that slot's last copy
//          is done, then queue copy + compute of i.
// The y of every expert from seq and pipe runs are compared bit for bit (same
// kernels, same inputs: any slot reuse hazard would show), and --verify dumps
// expert 0's x, h and y for the oracle check.
#include "fetcher.h"

namespace {

struct Gpu {
    kq_moe_desc d1;  // one-expert pool
    hipStream_t cs, ks;
    std::vector<uint8_t*> hbm;
    std::vector<hipEvent_t> copied, computed;  // per host slot / per HBM slot
    drv::DevBuf<uint16_t>* xh;
    drv::DevBuf<uint16_t>* h;
    drv::DevBuf<uint32_t>* idx;
    drv::DevBuf<float>* wgt;
    drv::DevBuf<float>* y;  // [n][hidden]
    size_t blob;

    void compute(uint32_t ds, int i) {
        const kq_stream_t k = reinterpret_cast<kq_stream_t>(ks);
        DRV_KQ(kq_moe_gate_up_swiglu(hbm[ds], &d1, idx->p, xh->p, h->p, 1, nullptr, 0, k));
        DRV_KQ(kq_moe_down_combine(hbm[ds], &d1, idx->p, wgt->p, h->p, y->p + (size_t)i * d1.hidden,
                                   KQ_F32, 1, nullptr, 0, k));
    }
    // host slot hs -> HBM slot ds, ordered after the compute that last read ds
    void copy(uint32_t hs, uint32_t ds, const char* src) {
        DRV_HIP(hipStreamWaitEvent(cs, computed[ds], 0));
        DRV_HIP(hipMemcpyAsync(hbm[ds], src, blob, hipMemcpyHostToDevice, cs));
        DRV_HIP(hipEventRecord(copied[hs], cs));
        DRV_HIP(hipStreamWaitEvent(ks, copied[hs], 0));
    }
};

}  // namespace

int main(int argc, char** argv) {
    const drv::Args args(argc, argv);
    if (args.flag("--help")) {
        printf("moepipe --store experts.bin [--experts n] [--depth d] [--workers w] [--reps r]\n"
               "        [--mode all|seq|io|pipe] [--hbm-slots n] [--warm] [--verify dir]\n");
        return 0;
    }
    const std::string store = args.str("--store", ""), mode = args.str("--mode", "all");
    const std::string vdir = args.str("--verify", "");
    const int depth = (int)std::max(1L, args.num("--depth", 3));
    const int workers = (int)std::max(1L, args.num("--workers", 4));
    const int reps = (int)std::max(1L, args.num("--reps", 3));
    const uint32_t nhbm = (uint32_t)std::max(2L, args.num("--hbm-slots", 2));
    const bool warm = args.flag("--warm");
    if (store.empty()) drv::die("--store is required");
    if (!(mode == "all" || mode == "seq" || mode == "io" || mode == "pipe")) drv::die("bad --mode");

    kq_moe_desc d;
    kq_moe_default_desc(&d);
    const size_t blob = d.blob;
    const int fd0 = open(store.c_str(), O_RDONLY);
    if (fd0 < 0) drv::die("cannot open " + store);
    const off_t fsize = lseek(fd0, 0, SEEK_END);
    close(fd0);
    const uint32_t nstore = (uint32_t)(fsize / (off_t)blob);
    if (nstore == 0) drv::die("store holds no whole expert");
    const int nexp = (int)std::min<long>(args.num("--experts", 288), nstore);
    auto expert_off = [&](int i) -> uint64_t {
        return ((uint64_t)i * 2654435761ull) % nstore * (uint64_t)blob;
    };

    const uint32_t nslots = (uint32_t)depth + 2;
    drv::Fetcher F(store, blob, nslots);

    // ---- GPU side: HBM slots, streams, events, the token
    Gpu g;
    g.d1 = d;
    g.d1.n_experts = 1;
    g.d1.top_k = 1;
    g.blob = blob;
    DRV_HIP(hipStreamCreate(&g.cs));
    DRV_HIP(hipStreamCreate(&g.ks));
    g.hbm.resize(nhbm);
    for (auto& p : g.hbm) DRV_HIP(hipMalloc(reinterpret_cast<void**>(&p), blob));
    g.copied.resize(nslots);
    g.computed.resize(nhbm);
    for (auto& e : g.copied) DRV_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    for (auto& e : g.computed) DRV_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    const uint32_t HID = d.hidden, INTER = d.inter;
    std::vector<float> x(HID);
    std::vector<uint16_t> xh(HID);
    for (uint32_t i = 0; i < HID; ++i) {  // the reference's token (moe-pipeline/src/main.mm:212-213)
        x[i] = 0.05f * ((int)(i % 17) - 8);
        xh[i] = drv::f2h(x[i]);
    }
    g.xh = new drv::DevBuf<uint16_t>(HID);
    g.xh->upload(xh.data(), HID);
    g.h = new drv::DevBuf<uint16_t>(INTER);
    g.idx = new drv::DevBuf<uint32_t>(1);
    g.idx->zero();
    g.wgt = new drv::DevBuf<float>(1);
    const float one = 1.0f;
    g.wgt->upload(&one, 1);
    g.y = new drv::DevBuf<float>((size_t)nexp * HID);

    F.read_blob(F.slot(0), expert_off(0));  // settles whether direct reads are taken
    printf("%s\n", kq_version());
    printf("store                 : %s (%u experts, %.2f GB)\n", store.c_str(), nstore, fsize / 1e9);
    printf("expert blob           : %.2f MB (gate/up/down, int4 g=64, bf16 scales)\n", blob / 1048576.0);
    if (F.direct())
        printf("page cache            : bypassed (O_DIRECT), readahead off\n");
    else
        printf("page cache            : %s (O_DIRECT refused: %s), readahead off\n",
               warm ? "in use (--warm)" : "store evicted before every run",
               F.direct_errno() ? strerror(F.direct_errno()) : "open");
    auto cold = [&]() {
        if (!F.direct() && !warm) F.evict();
    };
    printf("run                   : %d experts (%.2f GB) x %d reps, depth %d, %d readers, %u HBM slots\n\n",
           nexp, nexp * (double)blob / 1e9, reps, depth, workers, nhbm);

    // ---- GPU compute per expert, weights resident (rotating over the HBM slots)
    double t_comp = 0;
    {
        for (uint32_t s = 0; s < nhbm; ++s) {
            F.read_blob(F.slot(0), expert_off((int)s % nexp));
            DRV_HIP(hipMemcpy(g.hbm[s], F.slot(0), blob, hipMemcpyHostToDevice));
        }
        for (int w = 0; w < 4; ++w) g.compute((uint32_t)w % nhbm, 0);
        DRV_HIP(hipStreamSynchronize(g.ks));
        const int n = 40;
        double best = 1e30;
        for (int r = 0; r < 5; ++r) {
            const double t0 = drv::now_s();
            for (int i = 0; i < n; ++i) g.compute((uint32_t)i % nhbm, 0);
            DRV_HIP(hipStreamSynchronize(g.ks));
            best = std::min(best, (drv::now_s() - t0) / n);
        }
        t_comp = best;
        printf("GPU compute / expert  : %8.4f ms (%.1f GB/s over the blob, 2 launches)\n", t_comp * 1e3,
               blob / t_comp / 1e9);
    }

    struct Res {
        double wall = 1e30, busy = 0, exposed = 0;
    };
    auto run_seq = [&]() {
        Res r;
        r.exposed = 0;
        cold();
        const double t0 = drv::now_s();
        for (int i = 0; i < nexp; ++i) {
            const double r0 = drv::now_s();
            F.read_blob(F.slot(0), expert_off(i));
            const double dr = drv::now_s() - r0;
            r.busy += dr;
            r.exposed += dr;
            g.copy(0, (uint32_t)i % nhbm, F.slot(0));
            g.compute((uint32_t)i % nhbm, i);
            DRV_HIP(hipEventRecord(g.computed[(uint32_t)i % nhbm], g.ks));
            DRV_HIP(hipStreamSynchronize(g.ks));
        }
        r.wall = drv::now_s() - t0;
        return r;
    };
    auto run_io = [&]() {
        Res r;
        cold();
        F.reset();
        F.start(workers);
        const double t0 = drv::now_s();
        int issued = 0;
        for (; issued < (int)nslots && issued < nexp; ++issued) F.submit((uint32_t)issued, expert_off(issued), issued);
        for (int i = 0; i < nexp; ++i) {
            const uint32_t s = (uint32_t)i % nslots;
            F.wait_for(s, i);
            if (issued < nexp) {
                F.mark_empty(s);
                F.submit(s, expert_off(issued), issued);
                ++issued;
            }
        }
        r.wall = drv::now_s() - t0;
        F.stop_workers();
        r.busy = F.busy_s();
        return r;
    };
    auto run_pipe = [&]() {
        Res r;
        cold();
        F.reset();
        F.start(workers);
        const double t0 = drv::now_s();
        int issued = 0;
        for (; issued < depth && issued < nexp; ++issued)
            F.submit((uint32_t)issued % nslots, expert_off(issued), issued);
        for (int i = 0; i < nexp; ++i) {
            const uint32_t hs = (uint32_t)i % nslots, ds = (uint32_t)i % nhbm;
            r.exposed += F.wait_for(hs, i);
            if (issued < nexp) {  // refill before compute
                const uint32_t rs = (uint32_t)issued % nslots;
                DRV_HIP(hipEventSynchronize(g.copied[rs]));  // its last copy has left the slot
                F.mark_empty(rs);
                F.submit(rs, expert_off(issued), issued);
                ++issued;
            }
            g.copy(hs, ds, F.slot(hs));
            g.compute(ds, i);
            DRV_HIP(hipEventRecord(g.computed[ds], g.ks));
        }
        DRV_HIP(hipStreamSynchronize(g.ks));
        r.wall = drv::now_s() - t0;
        F.stop_workers();
        r.busy = F.busy_s();
        return r;
    };

    // ---- expert 0 for the oracle check
    if (!vdir.empty()) {
        F.read_blob(F.slot(0), expert_off(0));
        g.copy(0, 0, F.slot(0));
        g.compute(0, 0);
        DRV_HIP(hipEventRecord(g.computed[0], g.ks));
        DRV_HIP(hipStreamSynchronize(g.ks));
        const auto hh = g.h->download(INTER);
        const auto yy = g.y->download(HID);
        drv::write_file(vdir + "/x.f32", x.data(), HID * 4);
        drv::write_file(vdir + "/h.f16", hh.data(), INTER * 2);
        drv::write_file(vdir + "/y.f32", yy.data(), HID * 4);
        FILE* f = fopen((vdir + "/meta.txt").c_str(), "w");
        if (!f) drv::die("cannot write " + vdir);
        fprintf(f, "%llu %u %u %u\n", (unsigned long long)expert_off(0), HID, INTER, 64u);
        fclose(f);
        printf("dumped expert at byte offset %llu to %s\n", (unsigned long long)expert_off(0), vdir.c_str());
    }

    printf("\n%-28s %9s %10s %10s %10s %s\n", "driver", "wall", "GB/s", "tok/s", "read busy", "exposed IO");
    Res best[3];
    std::vector<float> y_seq, y_pipe;
    const bool all = mode == "all";
    const int want = mode == "seq" ? 0 : mode == "io" ? 1 : 2;
    // round-robin over the drivers (drift lands on none of them in particular)
    for (int rep = 0; rep < reps; ++rep)
        for (int k = 0; k < 3; ++k) {
            if (!all && k != want) continue;
            const Res x3 = k == 0 ? run_seq() : k == 1 ? run_io() : run_pipe();
            if (x3.wall < best[k].wall) best[k] = x3;
            if (k == 0 && y_seq.empty()) y_seq = g.y->download((size_t)nexp * HID);
            if (k == 2 && y_pipe.empty()) y_pipe = g.y->download((size_t)nexp * HID);
        }
    const char* nm[3] = {"seq  stop-and-wait", "io   reads only (ceiling)", "pipe stream+compute"};
    const double gb = nexp * (double)blob / 1e9, per_tok = 36.0 * 4.0;
    for (int k = 0; k < 3; ++k) {
        if (!all && k != want) continue;
        const Res& r = best[k];
        printf("  %-26s %7.3f s %7.2f GB/s %7.2f tok/s   busy %3.0f%%  exposed IO %6.3f s\n", nm[k], r.wall,
               gb / r.wall, nexp / per_tok / r.wall, 100.0 * r.busy / r.wall, r.exposed);
    }
    if (!y_seq.empty() && !y_pipe.empty()) {
        const bool same = memcmp(y_seq.data(), y_pipe.data(), y_seq.size() * 4) == 0;
        printf("\npipe outputs == seq outputs (bitwise, %d experts): %s\n", nexp, same ? "OK" : "FAIL");
        if (!same) return 1;
    }
    if (all) {
        printf("pipelined vs stop-and-wait : %.3fx\n", best[0].wall / best[2].wall);
        printf("pipelined vs reads-only    : %.1f%% of the read rate\n", 100.0 * best[1].wall / best[2].wall);
        printf("IO per expert %.3f ms vs compute %.4f ms\n", best[1].wall / nexp * 1e3, t_comp * 1e3);
    }
    delete g.xh;
    delete g.h;
    delete g.idx;
    delete g.wgt;
    delete g.y;
    for (auto p : g.hbm) (void)hipFree(p);
    return 0;
}
