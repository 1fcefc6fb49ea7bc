// fetcher.h -- reader threads that stream expert blobs from a store file into
// pinned host slots (the I/O stage of the moepipe driver).
//
// Counterpart of the reference's Fetcher (moe-pipeline/src/main.mm:74-154):
// a request queue served by worker threads, each request one pread of one
// blob into one slot, readiness published per slot. Here the slots are one
// hipHostMalloc'd block (pinned, so the copy engine DMAs them into HBM with
// hipMemcpyAsync) instead of shared CPU/GPU memory, and the page cache is
// bypassed with O_DIRECT (the store's blob size and offsets are 4 KiB
// multiples) where the kernel takes it for these pages, with readahead off
// either way.
//
// Readiness is published and tested under its own mutex (rmu): a worker that
// stored the slot's id and notified outside it could land between a waiter's
// test and its sleep, a missed wakeup.
#pragma once
#include <fcntl.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <condition_variable>
#include <mutex>
#include <queue>

#include "common.h"

namespace drv {

inline double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

class Fetcher {
   public:
    Fetcher(const std::string& path, size_t blob, uint32_t nslots) : blob_(blob), nslots_(nslots), ready_(nslots) {
        for (auto& r : ready_) r.store(-1);
        DRV_HIP(hipHostMalloc(reinterpret_cast<void**>(&base_), blob * nslots, hipHostMallocDefault));
        fd_ = open(path.c_str(), O_RDONLY | O_DIRECT);
        direct_ = fd_ >= 0;
        if (!direct_) fd_ = open(path.c_str(), O_RDONLY);
        if (fd_ < 0) die("cannot open " + path);
        (void)posix_fadvise(fd_, 0, 0, POSIX_FADV_RANDOM);  // no readahead
    }
    ~Fetcher() {
        stop_workers();
        close(fd_);
        (void)hipHostFree(base_);
    }
    Fetcher(const Fetcher&) = delete;
    Fetcher& operator=(const Fetcher&) = delete;

    bool direct() const { return direct_.load(); }
    int fd() const { return fd_; }
    uint32_t slots() const { return nslots_; }
    char* slot(uint32_t s) const { return base_ + (size_t)s * blob_; }

    // Reads one blob at `off` into `dst` on the calling thread. A direct
    // read the kernel refuses (EINVAL: the file system; EFAULT: the pinned
    // pages cannot be mapped for the device's DMA) makes the descriptor drop
    // O_DIRECT, and the read is made again buffered.
    void read_blob(char* dst, uint64_t off) {
        for (size_t got = 0; got < blob_;) {
            const ssize_t n = pread(fd_, dst + got, blob_ - got, (off_t)(off + got));
            if (n < 0 && direct_) {
                std::lock_guard<std::mutex> g(fmu_);
                if (direct_) {
                    direct_errno_ = errno;
                    (void)fcntl(fd_, F_SETFL, fcntl(fd_, F_GETFL) & ~O_DIRECT);
                    direct_ = false;
                }
                continue;
            }
            if (n <= 0)
                die("pread at " + std::to_string(off + got) + ": " + (n < 0 ? strerror(errno) : "end of file"));
            got += (size_t)n;
        }
    }
    // errno of the direct read that was refused (0: none was)
    int direct_errno() const { return direct_errno_; }
    // Drops the store's pages from the page cache (written back first), so
    // that buffered reads come off the device: what the reads of a run pay
    // when O_DIRECT is refused (each expert is read once per run, readahead
    // is off).
    void evict() const {
        (void)fsync(fd_);
        (void)posix_fadvise(fd_, 0, 0, POSIX_FADV_DONTNEED);
    }

    void start(int nworkers) {
        stop_ = false;
        for (int i = 0; i < nworkers; ++i) workers_.emplace_back([this] { loop(); });
    }
    void stop_workers() {
        {
            std::lock_guard<std::mutex> g(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
        workers_.clear();
    }
    void reset() {
        for (auto& r : ready_) r.store(-1);
        busy_s_ = 0;
        bytes_ = 0;
    }
    void mark_empty(uint32_t s) { ready_[s].store(-1); }
    void submit(uint32_t s, uint64_t off, int id) {
        {
            std::lock_guard<std::mutex> g(mu_);
            q_.push(Req{s, off, id});
        }
        cv_.notify_one();
    }
    // Blocks until slot s holds request `id`; returns the seconds blocked.
    double wait_for(uint32_t s, int id) {
        if (ready_[s].load(std::memory_order_acquire) == id) return 0.0;
        const double t0 = now_s();
        std::unique_lock<std::mutex> g(rmu_);
        done_cv_.wait(g, [&] { return ready_[s].load(std::memory_order_acquire) == id; });
        return now_s() - t0;
    }
    double busy_s() const { return busy_s_; }
    uint64_t bytes() const { return bytes_.load(); }

   private:
    struct Req {
        uint32_t slot;
        uint64_t off;
        int id;
    };
    void loop() {
        for (;;) {
            Req r;
            {
                std::unique_lock<std::mutex> g(mu_);
                cv_.wait(g, [&] { return stop_ || !q_.empty(); });
                if (q_.empty()) return;  // stopping with nothing left
                r = q_.front();
                q_.pop();
            }
            // wall time with at least one read outstanding (the device busy)
            if (inflight_.fetch_add(1) == 0) {
                std::lock_guard<std::mutex> g(bmu_);
                busy_t0_ = now_s();
            }
            read_blob(slot(r.slot), r.off);
            bytes_ += blob_;
            if (inflight_.fetch_sub(1) == 1) {
                std::lock_guard<std::mutex> g(bmu_);
                busy_s_ += now_s() - busy_t0_;
            }
            {
                std::lock_guard<std::mutex> g(rmu_);
                ready_[r.slot].store(r.id, std::memory_order_release);
            }
            done_cv_.notify_all();
        }
    }

    size_t blob_;
    uint32_t nslots_;
    char* base_ = nullptr;
    int fd_ = -1;
    std::atomic<bool> direct_{false};
    int direct_errno_ = 0;
    std::mutex fmu_;
    std::vector<std::atomic<int>> ready_;
    std::mutex mu_, rmu_, bmu_;
    std::condition_variable cv_, done_cv_;
    std::queue<Req> q_;
    std::vector<std::thread> workers_;
    bool stop_ = false;
    std::atomic<int> inflight_{0};
    double busy_s_ = 0, busy_t0_ = 0;
    std::atomic<uint64_t> bytes_{0};
};

}  // namespace drv
