// moepipe -- expert streaming from a store file into HBM, with each expert's
// gate/up + SwiGLU and down computed by libkq as it arrives. The experiment
// of moe-pipeline/src/main.mm (stop-and-wait, reads only, pipelined) on
// MI355X, where the path is disk -> pinned host memory -> HBM.
//
//   moepipe --store experts.bin [--experts 288] [--depth 3] [--workers 4]
//           [--reps 3] [--mode all|seq|io|pipe] [--hbm-slots 2] [--warm]
//           [--verify DIR]
//
// The store is the on-disk blob layout of gpt-oss-120b experts (14,024,704 B
// each, moe-fused/src/main.mm:23-25), any number of them. Step i streams
// store expert (i * 2654435761) mod n_store, a bijection on the store
// (2654435761 is prime), so no expert is read twice while --experts <=
// n_store.
//
// Stages of one expert (blob_ring.h holds the reader side):
//   disk -> pinned host slot   reader threads; O_DIRECT when the kernel takes
//                              it for pinned pages, else the store is evicted
//                              from the page cache before every run (unless
//                              --warm);
//   host slot -> HBM slot      hipMemcpyAsync on the copy stream, after the
//                              compute that last used the HBM slot (event);
//                              the copy's end is the host slot's drain event;
//   compute                    on the compute stream after the drain event:
//                              kq_moe_gate_up_swiglu + kq_moe_down_combine on
//                              the HBM slot as a one-expert pool (n_experts =
//                              top_k = 1, weight 1), y into a per-step row.
// The host thread waits only for reads to land.
//
//   seq  : read on the host thread, copy, compute, wait for the GPU; next.
//   io   : reads only, every host slot in flight (the rate the pipeline chases).
//   pipe : `depth` reads in flight: at step i take read i, open the read
//          window to i + depth (refill before compute), then queue copy and
//          compute of i.
// Every step's y of the seq and pipe runs are compared bit for bit (same
// kernels on the same bytes: a slot overwritten too early would show), and
// --verify dumps step 0's x, h and y for the oracle check.
#include "blob_ring.h"

namespace {

// The HBM side: slots, the two streams and the per-slot ordering events.
struct Device {
    kq_moe_desc one{};  // a one-expert pool
    size_t blob = 0;
    hipStream_t copy_q = nullptr, comp_q = nullptr;
    std::vector<uint8_t*> slot;
    std::vector<hipEvent_t> released;  // per HBM slot: the last compute that read it
    std::unique_ptr<drv::DevBuf<uint16_t>> xh, h;
    std::unique_ptr<drv::DevBuf<uint32_t>> idx;
    std::unique_ptr<drv::DevBuf<float>> wgt, y;  // y: [steps][hidden]

    Device(const kq_moe_desc& d, uint32_t nslot, int steps, const std::vector<uint16_t>& x16) : blob(d.blob) {
        one = d;
        one.n_experts = 1;
        one.top_k = 1;
        DRV_HIP(hipStreamCreate(&copy_q));
        DRV_HIP(hipStreamCreate(&comp_q));
        slot.resize(nslot);
        released.resize(nslot);
        for (uint32_t s = 0; s < nslot; ++s) {
            DRV_HIP(hipMalloc(reinterpret_cast<void**>(&slot[s]), blob));
            DRV_HIP(hipEventCreateWithFlags(&released[s], hipEventDisableTiming));
        }
        xh = std::make_unique<drv::DevBuf<uint16_t>>(d.hidden);
        xh->upload(x16.data(), d.hidden);
        h = std::make_unique<drv::DevBuf<uint16_t>>(d.inter);
        idx = std::make_unique<drv::DevBuf<uint32_t>>(1);
        idx->zero();
        wgt = std::make_unique<drv::DevBuf<float>>(1);
        const float w1 = 1.0f;
        wgt->upload(&w1, 1);
        y = std::make_unique<drv::DevBuf<float>>((size_t)std::max(1, steps) * d.hidden);
    }
    ~Device() {
        for (size_t s = 0; s < slot.size(); ++s) {
            (void)hipFree(slot[s]);
            (void)hipEventDestroy(released[s]);
        }
        (void)hipStreamDestroy(copy_q);
        (void)hipStreamDestroy(comp_q);
    }
    uint32_t nslot() const { return (uint32_t)slot.size(); }

    // The two MoE passes of one expert held in HBM slot s, y into row `row`.
    void compute(uint32_t s, int row) {
        const kq_stream_t q = reinterpret_cast<kq_stream_t>(comp_q);
        DRV_KQ(kq_moe_gate_up_swiglu(slot[s], &one, idx->p, xh->p, h->p, 1, nullptr, 0, q));
        DRV_KQ(kq_moe_down_combine(slot[s], &one, idx->p, wgt->p, h->p, y->p + (size_t)row * one.hidden, KQ_F32,
                                   1, nullptr, 0, q));
        DRV_HIP(hipEventRecord(released[s], comp_q));
    }
    // Host bytes -> HBM slot s (after the slot's last compute), `drain`
    // recorded at the copy's end, then the expert's compute after it.
    void land(const char* src, hipEvent_t drain, uint32_t s, int row) {
        DRV_HIP(hipStreamWaitEvent(copy_q, released[s], 0));
        DRV_HIP(hipMemcpyAsync(slot[s], src, blob, hipMemcpyHostToDevice, copy_q));
        DRV_HIP(hipEventRecord(drain, copy_q));
        DRV_HIP(hipStreamWaitEvent(comp_q, drain, 0));
        compute(s, row);
    }
};

struct RunStats {
    double wall = 1e30, busy = 0, exposed = 0;
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
    const int readers = (int)std::max(1L, args.num("--workers", 4));
    const int reps = (int)std::max(1L, args.num("--reps", 3));
    const uint32_t nhbm = (uint32_t)std::max(2L, args.num("--hbm-slots", 2));
    const bool warm = args.flag("--warm");
    if (store.empty()) drv::die("--store is required");
    if (!(mode == "all" || mode == "seq" || mode == "io" || mode == "pipe")) drv::die("bad --mode");

    kq_moe_desc d;
    kq_moe_default_desc(&d);
    const size_t blob = d.blob;
    uint32_t nstore = 0;
    {
        const int fd = open(store.c_str(), O_RDONLY);
        if (fd < 0) drv::die("cannot open " + store);
        nstore = (uint32_t)(lseek(fd, 0, SEEK_END) / (off_t)blob);
        close(fd);
    }
    if (nstore == 0) drv::die("store holds no whole expert");
    const int steps = (int)std::min<long>(args.num("--experts", 288), nstore);
    const std::function<uint64_t(int64_t)> where = [&](int64_t i) -> uint64_t {
        return ((uint64_t)i * 2654435761ull) % nstore * (uint64_t)blob;
    };

    drv::StoreFile file(store, blob);
    drv::BlobRing ring(file, (uint32_t)depth + 2);

    const uint32_t HID = d.hidden, INTER = d.inter;
    std::vector<float> x(HID);
    std::vector<uint16_t> x16(HID);
    for (uint32_t i = 0; i < HID; ++i) {  // the reference's token (moe-pipeline/src/main.mm:212-213)
        x[i] = 0.05f * ((int)(i % 17) - 8);
        x16[i] = drv::f2h(x[i]);
    }
    Device dev(d, nhbm, steps, x16);

    file.read(ring.host(0), where(0));  // settles whether direct reads are taken
    printf("%s\n", kq_version());
    printf("store                 : %s (%u experts, %.2f GB)\n", store.c_str(), nstore, nstore * (double)blob / 1e9);
    printf("expert blob           : %.2f MB (gate/up/down, int4 g=64, bf16 scales)\n", blob / 1048576.0);
    if (file.direct())
        printf("page cache            : bypassed (O_DIRECT), readahead off\n");
    else
        printf("page cache            : %s (O_DIRECT refused: %s), readahead off\n",
               warm ? "in use (--warm)" : "store evicted before every run",
               file.refused_errno() ? strerror(file.refused_errno()) : "open");
    const auto cold_start = [&]() {
        if (!file.direct() && !warm) file.evict();
    };
    printf("run                   : %d experts (%.2f GB) x %d reps, depth %d, %d readers, %u HBM slots\n\n",
           steps, steps * (double)blob / 1e9, reps, depth, readers, nhbm);

    // ---- GPU compute per expert with the blobs already in HBM
    double t_comp = 0;
    {
        for (uint32_t s = 0; s < dev.nslot(); ++s) {
            file.read(ring.host(0), where((int64_t)(s % (uint32_t)steps)));
            DRV_HIP(hipMemcpy(dev.slot[s], ring.host(0), blob, hipMemcpyHostToDevice));
        }
        for (int w = 0; w < 4; ++w) dev.compute((uint32_t)w % dev.nslot(), 0);
        DRV_HIP(hipStreamSynchronize(dev.comp_q));
        const int per = 40;
        for (int r = 0; r < 5; ++r) {
            const double t0 = drv::now_s();
            for (int i = 0; i < per; ++i) dev.compute((uint32_t)i % dev.nslot(), 0);
            DRV_HIP(hipStreamSynchronize(dev.comp_q));
            const double t = (drv::now_s() - t0) / per;
            t_comp = r == 0 ? t : std::min(t_comp, t);
        }
        printf("GPU compute / expert  : %8.4f ms (%.1f GB/s over the blob, 2 launches)\n", t_comp * 1e3,
               blob / t_comp / 1e9);
    }

    const auto stop_and_wait = [&]() {
        RunStats r;
        r.exposed = 0;
        cold_start();
        const double t0 = drv::now_s();
        for (int i = 0; i < steps; ++i) {
            const double r0 = drv::now_s();
            file.read(ring.host(0), where(i));
            const double dt = drv::now_s() - r0;
            r.busy += dt;
            r.exposed += dt;
            dev.land(ring.host(0), ring.drain(0), (uint32_t)i % dev.nslot(), i);
            DRV_HIP(hipStreamSynchronize(dev.comp_q));
        }
        r.wall = drv::now_s() - t0;
        return r;
    };
    const auto reads_only = [&]() {
        RunStats r;
        cold_start();
        const int64_t S = ring.size();
        const double t0 = drv::now_s();
        ring.start(steps, S, readers, where);
        for (int64_t i = 0; i < steps; ++i) {
            ring.take(i);
            ring.open_to(i + 1 + S);  // nothing copies out of the slot: it is free again
        }
        r.wall = drv::now_s() - t0;
        ring.finish();
        r.busy = ring.busy_s();
        return r;
    };
    const auto pipelined = [&]() {
        RunStats r;
        cold_start();
        const double t0 = drv::now_s();
        ring.start(steps, depth, readers, where);
        for (int64_t i = 0; i < steps; ++i) {
            r.exposed += ring.take(i);
            ring.open_to(i + 1 + depth);  // refill before compute
            dev.land(ring.host(i), ring.drain(i), (uint32_t)(i % dev.nslot()), (int)i);
        }
        DRV_HIP(hipStreamSynchronize(dev.comp_q));
        r.wall = drv::now_s() - t0;
        ring.finish();
        r.busy = ring.busy_s();
        return r;
    };

    // ---- step 0 for the oracle check
    if (!vdir.empty()) {
        file.read(ring.host(0), where(0));
        dev.land(ring.host(0), ring.drain(0), 0, 0);
        DRV_HIP(hipStreamSynchronize(dev.comp_q));
        const auto hh = dev.h->download(INTER);
        const auto yy = dev.y->download(HID);
        drv::write_file(vdir + "/x.f32", x.data(), HID * 4);
        drv::write_file(vdir + "/h.f16", hh.data(), INTER * 2);
        drv::write_file(vdir + "/y.f32", yy.data(), HID * 4);
        FILE* f = fopen((vdir + "/meta.txt").c_str(), "w");
        if (!f) drv::die("cannot write " + vdir);
        fprintf(f, "%llu %u %u %u\n", (unsigned long long)where(0), HID, INTER, 64u);
        fclose(f);
        printf("dumped expert at byte offset %llu to %s\n", (unsigned long long)where(0), vdir.c_str());
    }

    printf("\n%-28s %9s %10s %10s %10s %s\n", "driver", "wall", "GB/s", "tok/s", "read busy", "exposed IO");
    const char* names[3] = {"seq  stop-and-wait", "io   reads only (ceiling)", "pipe stream+compute"};
    const bool all = mode == "all";
    const int only = mode == "seq" ? 0 : mode == "io" ? 1 : 2;
    RunStats best[3];
    std::vector<float> y_seq, y_pipe;
    // the drivers take turns in every rep, so drift is shared
    for (int rep = 0; rep < reps; ++rep)
        for (int k = 0; k < 3; ++k) {
            if (!all && k != only) continue;
            const RunStats got = k == 0 ? stop_and_wait() : k == 1 ? reads_only() : pipelined();
            if (got.wall < best[k].wall) best[k] = got;
            if (k == 0 && y_seq.empty()) y_seq = dev.y->download((size_t)steps * HID);
            if (k == 2 && y_pipe.empty()) y_pipe = dev.y->download((size_t)steps * HID);
        }
    const double gb = steps * (double)blob / 1e9, experts_per_token = 36.0 * 4.0;
    for (int k = 0; k < 3; ++k) {
        if (!all && k != only) continue;
        const RunStats& r = best[k];
        printf("  %-26s %7.3f s %7.2f GB/s %7.2f tok/s   busy %3.0f%%  exposed IO %6.3f s\n", names[k], r.wall,
               gb / r.wall, steps / experts_per_token / r.wall, 100.0 * r.busy / r.wall, r.exposed);
    }
    if (!y_seq.empty() && !y_pipe.empty()) {
        const bool same = memcmp(y_seq.data(), y_pipe.data(), y_seq.size() * 4) == 0;
        printf("\npipe outputs == seq outputs (bitwise, %d experts): %s\n", steps, same ? "OK" : "FAIL");
        if (!same) return 1;
    }
    if (all) {
        printf("pipelined vs stop-and-wait : %.3fx\n", best[0].wall / best[2].wall);
        printf("pipelined vs reads-only    : %.1f%% of the read rate\n", 100.0 * best[1].wall / best[2].wall);
        printf("IO per expert %.3f ms vs compute %.4f ms\n", best[1].wall / steps * 1e3, t_comp * 1e3);
    }
    return 0;
}
