// common.h -- shared plumbing of the C++ host drivers (int4gemv, vqgemv,
// moefused). The drivers mirror the reference's Objective-C++ harnesses
// (int4-gemv/src/main.mm, vq-gemv/src/main.mm, moe-fused/src/main.mm): the
// same arguments, seeded buffers in the same layouts, weight copies rotated
// per dispatch, every variant checked before anything is timed, round-robin
// timing of all variants, and the same report. They call libkq through its C
// ABI only (include/kq.h); device memory comes from hipMalloc.
//
// Verification, as in the reference harnesses, compares every variant with an
// fp64 host evaluation of the same formula on the same buffers (max |d| /
// max |y| < 2e-3, int4-gemv/src/main.mm:475-479); the drivers exit 1 on a
// mismatch. That evaluation only checks: no result a driver reports comes
// from it. The test suite additionally checks the tensors a --dump run writes
// against the repository's CPU oracle.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <thread>
#include <vector>

#include "kq.h"

namespace drv {

[[noreturn]] inline void die(const std::string& what) {
    fprintf(stderr, "FATAL: %s\n", what.c_str());
    exit(1);
}

#define DRV_HIP(x)                                                                  \
    do {                                                                            \
        const hipError_t e_ = (x);                                                  \
        if (e_ != hipSuccess) drv::die(std::string(#x) + ": " + hipGetErrorString(e_)); \
    } while (0)

#define DRV_KQ(x)                                                                        \
    do {                                                                                 \
        const kq_status s_ = (x);                                                        \
        if (s_ != KQ_OK) drv::die(std::string(#x) + ": " + kq_status_str(s_));           \
    } while (0)

inline uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
inline float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
inline float bf2f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }
inline uint16_t f2bf(float f) {  // round to nearest even
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// f(a, b) over [0, n) split across the host's threads (the reference's par(),
// moe-fused/src/main.mm:64-73).
template <typename F>
inline void par(size_t n, F f) {
    const size_t nt = std::max(1u, std::thread::hardware_concurrency());
    const size_t c = (n + nt - 1) / nt;
    std::vector<std::thread> th;
    for (size_t i = 0; i < nt && i * c < n; ++i) th.emplace_back(f, i * c, std::min(n, i * c + c));
    for (auto& t : th) t.join();
}

// "--name value" arguments; flags take no value.
struct Args {
    std::vector<std::string> a;
    Args(int argc, char** argv) : a(argv + 1, argv + argc) {}
    const char* find(const char* n) const {
        for (size_t i = 0; i + 1 < a.size(); ++i)
            if (a[i] == n) return a[i + 1].c_str();
        return nullptr;
    }
    bool flag(const char* n) const { return std::find(a.begin(), a.end(), n) != a.end(); }
    long num(const char* n, long d) const {
        const char* v = find(n);
        return v ? atol(v) : d;
    }
    std::string str(const char* n, const std::string& d) const {
        const char* v = find(n);
        return v ? std::string(v) : d;
    }
};

template <typename T>
struct DevBuf {
    T* p = nullptr;
    size_t n = 0;
    explicit DevBuf(size_t count) : n(count) {
        DRV_HIP(hipMalloc(reinterpret_cast<void**>(&p), std::max<size_t>(1, n) * sizeof(T)));
    }
    ~DevBuf() { (void)hipFree(p); }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    size_t bytes() const { return n * sizeof(T); }
    void upload(const T* h, size_t count, size_t at = 0) {
        DRV_HIP(hipMemcpy(p + at, h, count * sizeof(T), hipMemcpyHostToDevice));
    }
    std::vector<T> download(size_t count, size_t at = 0) const {
        std::vector<T> h(count);
        DRV_HIP(hipMemcpy(h.data(), p + at, count * sizeof(T), hipMemcpyDeviceToHost));
        return h;
    }
    void zero() { DRV_HIP(hipMemset(p, 0, bytes())); }
};

inline void write_file(const std::string& path, const void* p, size_t n) {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) die("cannot write " + path);
    if (fwrite(p, 1, n, f) != n) die("short write " + path);
    fclose(f);
}

// Copies of a weight set rotated per dispatch so that consecutive dispatches
// never find their weights in L2 or the 256 MB MALL (the reference rotates
// over 192 MB against the M4's 8 MB SLC, int4-gemv/src/main.mm:164-176).
inline uint32_t n_copies(size_t set_bytes, size_t rot_bytes) {
    return (uint32_t)std::min<size_t>(64, std::max<size_t>(1, (rot_bytes + set_bytes - 1) / set_bytes));
}

// One timed variant: enc(stream, rep) launches dispatch `rep` of a span.
struct Variant {
    std::string name;
    std::function<void(hipStream_t, int)> enc;
    double bytes = 0;  // per dispatch
    bool check = true;
    double best_s = 0, med_s = 0, relerr = 0;
    int launches = 1;  // kernel launches per dispatch (reported)
};

// Dispatches per span chosen so a span lasts ~5 ms (at most 64), as the
// reference does (int4-gemv/src/main.mm:453-460).
inline int probe_repeat(Variant& v, hipStream_t s) {
    hipEvent_t e0, e1;
    DRV_HIP(hipEventCreate(&e0));
    DRV_HIP(hipEventCreate(&e1));
    v.enc(s, 0);
    DRV_HIP(hipStreamSynchronize(s));
    DRV_HIP(hipEventRecord(e0, s));
    v.enc(s, 0);
    DRV_HIP(hipEventRecord(e1, s));
    DRV_HIP(hipEventSynchronize(e1));
    float ms = 0;
    DRV_HIP(hipEventElapsedTime(&ms, e0, e1));
    DRV_HIP(hipEventDestroy(e0));
    DRV_HIP(hipEventDestroy(e1));
    return (int)std::min(64.0, std::max(1.0, std::ceil(5.0 / std::max(ms, 1e-4f))));
}

// Round-robin timing (int4-gemv/src/main.mm:496-521): every variant once per
// round, so clock drift is shared; per-dispatch best and median.
inline void time_round_robin(std::vector<Variant>& vars, hipStream_t s, int repeat, int warmup,
                             int iters) {
    hipEvent_t e0, e1;
    DRV_HIP(hipEventCreate(&e0));
    DRV_HIP(hipEventCreate(&e1));
    for (auto& v : vars)
        for (int i = 0; i < warmup; ++i)
            for (int r = 0; r < repeat; ++r) v.enc(s, r);
    DRV_HIP(hipStreamSynchronize(s));
    std::vector<std::vector<double>> samples(vars.size());
    for (int it = 0; it < iters; ++it)
        for (size_t i = 0; i < vars.size(); ++i) {
            DRV_HIP(hipEventRecord(e0, s));
            for (int r = 0; r < repeat; ++r) vars[i].enc(s, r);
            DRV_HIP(hipEventRecord(e1, s));
            DRV_HIP(hipEventSynchronize(e1));
            float ms = 0;
            DRV_HIP(hipEventElapsedTime(&ms, e0, e1));
            samples[i].push_back(ms * 1e-3 / repeat);
        }
    for (size_t i = 0; i < vars.size(); ++i) {
        std::sort(samples[i].begin(), samples[i].end());
        vars[i].best_s = samples[i].front();
        vars[i].med_s = samples[i][samples[i].size() / 2];
    }
    DRV_HIP(hipEventDestroy(e0));
    DRV_HIP(hipEventDestroy(e1));
}

// max |got - ref| / max |ref| (the reference's metric).
template <typename F, typename G>
inline double rel_inf(size_t n, F got, G ref) {
    double mx = 0, md = 0;
    for (size_t i = 0; i < n; ++i) {
        mx = std::max(mx, std::fabs(ref(i)));
        md = std::max(md, std::fabs(got(i) - ref(i)));
    }
    return md / std::max(mx, 1e-30);
}

constexpr double kPeakGBs = 8000.0;  // MI355X HBM3E

inline void print_table(const std::vector<Variant>& vars, double ceil_gbs) {
    const char* rule = "-----------------------------------------------------------------------------------------------\n";
    printf("\n%-40s %9s %9s %9s %7s %7s %9s\n", "variant", "GB/s", "GB/s(med)", "us", "% peak",
           "% ceil", "err/|ref|");
    printf("%s", rule);
    for (const auto& v : vars) {
        const double g = v.bytes / v.best_s / 1e9, gm = v.bytes / v.med_s / 1e9;
        printf("  %-38s %9.1f %9.1f %9.3f %7.1f %7.1f", v.name.c_str(), g, gm, v.best_s * 1e6,
               100.0 * g / kPeakGBs, ceil_gbs > 0 ? 100.0 * g / ceil_gbs : 0.0);
        if (v.check)
            printf(" %9.1e\n", v.relerr);
        else
            printf(" %9s\n", "-");
    }
    printf("%s", rule);
}

}  // namespace drv
