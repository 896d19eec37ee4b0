// Host side of the staged boundary copies: the chunk plan over the pinned
// staging slots and a parallel memcpy on persistent worker threads.  No HIP
// here, so the CPU test (tests/host_copy_test.cpp) compiles it with g++.
//
// Why: a DMA from pageable memory runs at the rate of the HIP runtime's own
// staging (17-29 GB/s measured on MI355X), a DMA from pinned memory at
// ~57 GB/s, and one host thread copies pageable -> pinned at ~30 GB/s (four
// at ~75 GB/s).  So the boundary copies go through a ring of pinned slots
// filled (or drained) by a few host threads while the previous slot's DMA
// runs.
#pragma once

#include <algorithm>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

namespace camel_hip {

// Calls fn(index, offset, size) for the chunks of a staged copy of `bytes`
// in slot-sized pieces: offsets ascending and contiguous, every size in
// (0, slot_bytes], the sizes summing to bytes (nothing for bytes == 0).
// (Chunks ramping 1, 2, 4 MiB up and down at the ends, to shorten the
// pipeline's fill and drain, measured no faster on MI355X.)
template <class Fn> void for_each_chunk(size_t bytes, size_t slot_bytes, Fn &&fn) {
    size_t index = 0;
    for (size_t off = 0; off < bytes; off += slot_bytes, ++index)
        fn(index, off, std::min(slot_bytes, bytes - off));
}

// memcpy split over the calling thread and `workers` persistent threads.
// One copy runs at a time (callers serialise: the library holds its mutex);
// pieces below `min_piece` bytes are not split further.  The library's pool
// is never destroyed (its threads wait on it until the process ends); a
// pool that is destroyed stops and joins its threads first.
class CopyPool {
  public:
    explicit CopyPool(int workers, size_t min_piece = size_t(1) << 20)
        : workers_(std::max(0, workers)), min_piece_(std::max<size_t>(min_piece, 1)) {
        for (int i = 0; i < workers_; ++i) threads_.emplace_back([this, i] { run(i + 1); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lock(m_);
            stop_ = true;
        }
        work_.notify_all();
        for (auto &t : threads_) t.join();
    }
    CopyPool(const CopyPool &) = delete;
    CopyPool &operator=(const CopyPool &) = delete;

    // Pieces a copy of n bytes is split into (1 .. workers + 1); piece p
    // covers [begin(n, p), begin(n, p + 1)), boundaries on 4 KiB multiples.
    int pieces(size_t n) const {
        const size_t by_size = n / min_piece_;
        return (int)std::max<size_t>(1, std::min<size_t>(by_size, (size_t)workers_ + 1));
    }
    static size_t begin(size_t n, int parts, int p) {
        if (p >= parts) return n;
        const size_t per = ((n / parts) + 4095) & ~size_t(4095);
        return std::min(n, per * (size_t)p);
    }

    void copy(void *dst, const void *src, size_t n) {
        const int parts = pieces(n);
        if (parts == 1) {
            if (n) std::memcpy(dst, src, n);
            return;
        }
        {
            std::lock_guard<std::mutex> lock(m_);
            dst_ = static_cast<char *>(dst);
            src_ = static_cast<const char *>(src);
            n_ = n;
            parts_ = parts;
            pending_ = parts - 1;
            ++generation_;
        }
        work_.notify_all();
        piece(0);
        std::unique_lock<std::mutex> lock(m_);
        done_.wait(lock, [this] { return pending_ == 0; });
    }

  private:
    void piece(int p) {
        const size_t a = begin(n_, parts_, p), b = begin(n_, parts_, p + 1);
        if (b > a) std::memcpy(dst_ + a, src_ + a, b - a);
    }
    void run(int id) {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lock(m_);
        for (;;) {
            work_.wait(lock, [&] { return generation_ != seen || stop_; });
            if (stop_) return;
            seen = generation_;
            if (id >= parts_) continue;
            lock.unlock();
            piece(id);
            lock.lock();
            if (--pending_ == 0) done_.notify_one();
        }
    }

    const int workers_;
    const size_t min_piece_;
    std::mutex m_;
    std::condition_variable work_, done_;
    std::vector<std::thread> threads_;
    bool stop_ = false;
    uint64_t generation_ = 0;
    int pending_ = 0;
    int parts_ = 1;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t n_ = 0;
};

} // namespace camel_hip
