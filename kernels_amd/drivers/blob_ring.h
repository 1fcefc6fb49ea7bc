// blob_ring.h -- the I/O stage of the moepipe driver: expert blobs read from
// a store file into a ring of pinned host slots by reader threads, under a
// read window that the consumer advances.
//
// The reference's I/O stage (moe-pipeline/src/main.mm:74-154) serves a
// request queue. This one has no queue and no locks:
//
//  * A run is a fixed sequence of n reads; read i takes the blob at byte
//    offset off(i) into slot i % S. Readers claim reads in order from one
//    atomic ticket counter and leave when the tickets run out.
//  * The consumer owns a window word: read i may start once window > i. After
//    the consumer has taken read i it opens the window to i + 1 + lead, before
//    it queues any work for read i (refill before compute): `lead` reads stay
//    in flight while the GPU works.
//  * A slot may be overwritten only after the HIP copy that last read it has
//    finished. The consumer records that copy's end as the slot's drain event;
//    the reader of the next blob for the slot waits for that event itself, so
//    the consumer thread never blocks on the DMA engine. The event is recorded
//    before the window opens past the slot's next read whenever S >= lead + 1
//    (read i + lead goes to the slot of read i + lead - S <= i - 1, whose copy
//    was queued at an earlier step); S = lead + 2 leaves one slot for the copy
//    in flight.
//  * Each slot has a completion word holding the id of the read that last
//    landed in it. The reader stores it with release order and wakes waiters;
//    the consumer waits with std::atomic::wait, which compares the word again
//    inside the futex wait, so a store between the consumer's test and its
//    sleep cannot be missed.
//  * Every read stores its own [start, end) host times in its own cell. A
//    run's busy time (wall time with at least one read in progress) is the
//    measure of the union of those intervals, computed after the readers have
//    joined.
#pragma once
#include <fcntl.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <functional>
#include <memory>

#include "common.h"

namespace drv {

inline double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// The store file. Reads bypass the page cache with O_DIRECT where the kernel
// takes it (the blob size and offsets are 4 KiB multiples); a direct read
// the kernel refuses (EINVAL: the file system; EFAULT: the destination is
// pinned for the device's DMA and cannot be mapped) clears O_DIRECT on the
// descriptor once, for every reader, and is made again buffered. Readahead
// is off either way.
class StoreFile {
   public:
    StoreFile(const std::string& path, size_t blob) : blob_(blob) {
        fd_ = open(path.c_str(), O_RDONLY | O_DIRECT);
        bool direct = fd_ >= 0;
        if (!direct) fd_ = open(path.c_str(), O_RDONLY);
        if (fd_ < 0) die("cannot open " + path);
        direct_.store(direct);
        (void)posix_fadvise(fd_, 0, 0, POSIX_FADV_RANDOM);
    }
    ~StoreFile() { close(fd_); }
    StoreFile(const StoreFile&) = delete;
    StoreFile& operator=(const StoreFile&) = delete;

    size_t blob() const { return blob_; }
    bool direct() const { return direct_.load(); }
    int refused_errno() const { return refused_errno_.load(); }

    void read(char* dst, uint64_t off) {
        size_t got = 0;
        while (got < blob_) {
            const ssize_t n = pread(fd_, dst + got, blob_ - got, (off_t)(off + got));
            if (n > 0) {
                got += (size_t)n;
                continue;
            }
            if (n < 0 && direct_.load()) {
                drop_direct(errno);
                continue;
            }
            die("pread at " + std::to_string(off + got) + ": " + (n < 0 ? strerror(errno) : "end of file"));
        }
    }
    // Writes back and drops the store's cached pages, so that buffered reads
    // come off the device (each blob is read once per run, readahead is off).
    void evict() const {
        (void)fsync(fd_);
        (void)posix_fadvise(fd_, 0, 0, POSIX_FADV_DONTNEED);
    }

   private:
    void drop_direct(int err) {
        bool expect = true;
        if (direct_.compare_exchange_strong(expect, false)) {
            refused_errno_.store(err);
            (void)fcntl(fd_, F_SETFL, fcntl(fd_, F_GETFL) & ~O_DIRECT);
        }
    }
    size_t blob_;
    int fd_ = -1;
    std::atomic<bool> direct_{false};
    std::atomic<int> refused_errno_{0};
};

class BlobRing {
   public:
    // S pinned host slots of one blob each (hipHostMalloc: the copy engine
    // reads them directly), and one drain event per slot.
    BlobRing(StoreFile& file, uint32_t nslots) : file_(file), slots_(nslots) {
        const size_t blob = file.blob();
        DRV_HIP(hipHostMalloc(reinterpret_cast<void**>(&pinned_), blob * nslots, hipHostMallocDefault));
        for (uint32_t s = 0; s < nslots; ++s) {
            slots_[s].host = pinned_ + (size_t)s * blob;
            DRV_HIP(hipEventCreateWithFlags(&slots_[s].drain, hipEventDisableTiming));
        }
    }
    ~BlobRing() {
        finish();
        for (auto& s : slots_) (void)hipEventDestroy(s.drain);
        (void)hipHostFree(pinned_);
    }
    BlobRing(const BlobRing&) = delete;
    BlobRing& operator=(const BlobRing&) = delete;

    uint32_t size() const { return (uint32_t)slots_.size(); }
    char* host(int64_t i) const { return slots_[(size_t)(i % (int64_t)slots_.size())].host; }
    // The event the consumer records after the copy that reads read i's slot.
    hipEvent_t drain(int64_t i) const { return slots_[(size_t)(i % (int64_t)slots_.size())].drain; }

    // Starts `readers` threads over reads 0 .. n-1 with reads 0 .. window-1
    // open at once.
    void start(int64_t n, int64_t window, int readers, std::function<uint64_t(int64_t)> off) {
        finish();
        n_ = n;
        off_ = std::move(off);
        next_.store(0);
        window_.store(window);
        cells_.assign((size_t)n, Cell{});
        for (auto& s : slots_) s.done.store(-1);
        for (int r = 0; r < readers; ++r) threads_.emplace_back([this] { serve(); });
    }
    // Blocks until read i has landed; returns the seconds it waited.
    double take(int64_t i) {
        std::atomic<int64_t>& w = slots_[(size_t)(i % (int64_t)slots_.size())].done;
        int64_t v = w.load(std::memory_order_acquire);
        if (v == i) return 0.0;
        const double t0 = now_s();
        while (v != i) {
            w.wait(v, std::memory_order_acquire);
            v = w.load(std::memory_order_acquire);
        }
        return now_s() - t0;
    }
    // Lets reads up to end - 1 start (the window only grows).
    void open_to(int64_t end) {
        int64_t cur = window_.load();
        while (cur < end && !window_.compare_exchange_weak(cur, end)) {
        }
        window_.notify_all();
    }
    // Joins the readers of the current run (every read has been taken or the
    // window is open to the end).
    void finish() {
        if (threads_.empty()) return;
        open_to(n_);
        for (auto& t : threads_) t.join();
        threads_.clear();
    }
    // Wall time of the finished run with at least one read in progress.
    double busy_s() const {
        std::vector<Cell> c(cells_);
        std::sort(c.begin(), c.end(), [](const Cell& a, const Cell& b) { return a.t0 < b.t0; });
        double busy = 0, lo = 0, hi = -1;
        for (const Cell& x : c) {
            if (x.t1 <= x.t0) continue;
            if (x.t0 > hi) {
                if (hi > lo) busy += hi - lo;
                lo = x.t0;
                hi = x.t1;
            } else {
                hi = std::max(hi, x.t1);
            }
        }
        if (hi > lo) busy += hi - lo;
        return busy;
    }

   private:
    struct Slot {
        char* host = nullptr;
        hipEvent_t drain = nullptr;
        std::atomic<int64_t> done{-1};
    };
    struct Cell {
        double t0 = 0, t1 = 0;
    };
    void serve() {
        for (;;) {
            const int64_t i = next_.fetch_add(1);
            if (i >= n_) return;
            int64_t w = window_.load(std::memory_order_acquire);
            while (w <= i) {
                window_.wait(w, std::memory_order_acquire);
                w = window_.load(std::memory_order_acquire);
            }
            Slot& s = slots_[(size_t)(i % (int64_t)slots_.size())];
            DRV_HIP(hipEventSynchronize(s.drain));  // the copy out of this slot's last blob
            const double t0 = now_s();
            file_.read(s.host, off_(i));
            cells_[(size_t)i] = Cell{t0, now_s()};
            s.done.store(i, std::memory_order_release);
            s.done.notify_all();
        }
    }

    StoreFile& file_;
    char* pinned_ = nullptr;
    std::vector<Slot> slots_;
    std::vector<std::thread> threads_;
    std::vector<Cell> cells_;
    std::function<uint64_t(int64_t)> off_;
    int64_t n_ = 0;
    std::atomic<int64_t> next_{0};
    std::atomic<int64_t> window_{0};
};

}  // namespace drv
