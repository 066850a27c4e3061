// tk_staging.h -- host side of the host-to-host entry points: pinned
// staging buffers and a small pool of copy threads, so that the CPU copies
// between the caller's (pageable) buffers and the pinned staging overlap
// the DMA transfers of neighbouring chunks (internal to libtoktier_hip).
//
// The reference's fused lane stages the request the same way (the UTF-8
// bytes copied into a pinned buffer, then a non-blocking host-to-device
// copy; src/toktier/engine/gpu/encoder.py:462-467, :566-567); here the
// copies are split into chunks over several threads and pipelined with the
// transfers in both directions.
#pragma once
#include <hip/hip_runtime.h>
#include <sched.h>

#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace tk {

// Runs jobs of n numbered chunks on a few worker threads; chunks are handed
// out in increasing order (one atomic counter), so chunk k starts no later
// than chunk k+1.
class CopyPool {
 public:
  explicit CopyPool(int threads) {
    for (int i = 0; i < threads; ++i) th_.emplace_back([this] { loop(); });
  }
  ~CopyPool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : th_) t.join();
  }
  CopyPool(const CopyPool&) = delete;
  CopyPool& operator=(const CopyPool&) = delete;

  int threads() const { return (int)th_.size(); }

  // Starts fn(0..n-1) on the workers and returns; wait() ends the job.
  void start(size_t n, std::function<void(size_t)> fn) {
    {
      std::lock_guard<std::mutex> lk(mu_);
      fn_ = std::move(fn);
      n_ = n;
      finished_ = 0;
      next_.store(0, std::memory_order_relaxed);
      ++gen_;
    }
    cv_.notify_all();
  }
  void wait() {
    std::unique_lock<std::mutex> lk(mu_);
    done_cv_.wait(lk, [&] { return finished_ >= n_; });
  }

 private:
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      std::function<void(size_t)> fn;
      size_t n;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
        if (stop_) return;
        seen = gen_;
        fn = fn_;
        n = n_;
      }
      size_t done = 0;
      for (size_t k; (k = next_.fetch_add(1, std::memory_order_relaxed)) < n;) {
        fn(k);
        ++done;
      }
      std::lock_guard<std::mutex> lk(mu_);
      finished_ += done;
      if (finished_ >= n_) done_cv_.notify_all();
    }
  }
  std::vector<std::thread> th_;
  std::mutex mu_;
  std::condition_variable cv_, done_cv_;
  std::function<void(size_t)> fn_;
  size_t n_ = 0;
  size_t finished_ = 0;
  std::atomic<size_t> next_{0};
  uint64_t gen_ = 0;
  bool stop_ = false;
};

// copy threads for a process allowed `cpus` CPUs: half of them, 1..8
inline int copy_threads() {
  cpu_set_t set;
  int cpus = 8;
  if (sched_getaffinity(0, sizeof set, &set) == 0) cpus = CPU_COUNT(&set);
  const int n = cpus / 2;
  return n < 1 ? 1 : n > 8 ? 8 : n;
}

// Pinned host memory (hipHostMalloc), grown on demand.
struct PinnedBuf {
  uint8_t* p = nullptr;
  size_t n = 0;
  ~PinnedBuf() { reset(); }
  void reset() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    n = 0;
  }
  hipError_t ensure(size_t bytes) {
    if (bytes <= n) return hipSuccess;
    reset();
    void* q = nullptr;
    hipError_t e = hipHostMalloc(&q, bytes, hipHostMallocDefault);
    if (e == hipSuccess) {
      p = static_cast<uint8_t*>(q);
      n = bytes;
    }
    return e;
  }
};

// Chunks of a transfer of `bytes`: at least `min_chunk` bytes each and at
// most `max_chunks` of them.
inline size_t chunk_bytes(size_t bytes, size_t min_chunk, size_t max_chunks) {
  size_t c = min_chunk;
  while ((bytes + c - 1) / c > max_chunks) c <<= 1;
  return c;
}

}  // namespace tk
