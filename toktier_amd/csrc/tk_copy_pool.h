// tk_copy_pool.h -- the copy threads of the host-to-host entry points
// (internal to libtoktier_hip; no HIP dependency, so the pool is also
// built on its own by a CPU stress test under ThreadSanitizer).
#pragma once
#include <sched.h>

#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace tk {

// Runs jobs of n numbered chunks on a few worker threads and the calling
// thread. A chunk is claimed from one counter that holds the job's
// generation beside the next chunk number, so a worker that wakes late
// cannot take a chunk of a later job. After a job a worker keeps polling
// for the next one for SPIN before it sleeps: calls that come back to back
// find the workers awake (a wake-up from sleep costs tens of microseconds,
// as long as the copy itself).
class CopyPool {
 public:
  static constexpr std::chrono::microseconds SPIN{1000};

  explicit CopyPool(int threads) {
    for (int i = 0; i < threads; ++i) th_.emplace_back([this] { loop(); });
  }
  ~CopyPool() {
    {
      std::lock_guard<std::mutex> lk(mu_);
      stop_.store(true);
    }
    cv_.notify_all();
    for (auto& t : th_) t.join();
  }
  CopyPool(const CopyPool&) = delete;
  CopyPool& operator=(const CopyPool&) = delete;

  int threads() const { return (int)th_.size(); }

  // Runs fn(0..n-1) and returns once every chunk has run. Calls do not
  // overlap (the engine's mutex holds one call at a time).
  void run(size_t n, const std::function<void(size_t)>& fn) {
    if (n == 0) return;
    const uint64_t g = (gen_.load(std::memory_order_relaxed) + 1) & 0xFFFFFFFFu;
    Job& j = jobs_[g & 1];
    j.fn.store(&fn, std::memory_order_relaxed);
    j.n.store(n, std::memory_order_relaxed);
    done_.store(0, std::memory_order_relaxed);
    ctr_.store(g << 32, std::memory_order_release);
    gen_.store(g);  // seq_cst: ordered against the workers' parked_ count
    if (parked_.load() > 0) {
      std::lock_guard<std::mutex> lk(mu_);
      cv_.notify_all();
    }
    size_t k;
    while (claim(g, n, &k)) {
      fn(k);
      done_.fetch_add(1, std::memory_order_acq_rel);
    }
    while (done_.load(std::memory_order_acquire) < n) std::this_thread::yield();
  }

 private:
  struct Job {
    std::atomic<const std::function<void(size_t)>*> fn{nullptr};
    std::atomic<size_t> n{0};
  };

  // takes the next chunk of job g, if job g is still the current one
  bool claim(uint64_t g, size_t n, size_t* k) {
    uint64_t v = ctr_.load(std::memory_order_acquire);
    for (;;) {
      if ((v >> 32) != g || (v & 0xFFFFFFFFu) >= n) return false;
      if (ctr_.compare_exchange_weak(v, v + 1, std::memory_order_acq_rel,
                                     std::memory_order_acquire)) {
        *k = (size_t)(v & 0xFFFFFFFFu);
        return true;
      }
    }
  }

  void loop() {
    uint64_t seen = 0;
    for (;;) {
      uint64_t g = gen_.load(std::memory_order_acquire);
      if (g == seen) {
        const auto until = std::chrono::steady_clock::now() + SPIN;
        while ((g = gen_.load(std::memory_order_acquire)) == seen &&
               !stop_.load(std::memory_order_relaxed) &&
               std::chrono::steady_clock::now() < until)
          std::this_thread::yield();
        if (g == seen) {
          std::unique_lock<std::mutex> lk(mu_);
          parked_.fetch_add(1);
          cv_.wait(lk, [&] { return stop_.load() || gen_.load() != seen; });
          parked_.fetch_sub(1);
        }
        if (stop_.load()) return;
        continue;
      }
      seen = g;
      const Job& j = jobs_[g & 1];
      const std::function<void(size_t)>* fn = j.fn.load(std::memory_order_relaxed);
      const size_t n = j.n.load(std::memory_order_relaxed);
      size_t k;
      // a claim succeeds only while job g is current, so fn and n are its own
      while (claim(g, n, &k)) {
        (*fn)(k);
        done_.fetch_add(1, std::memory_order_acq_rel);
      }
    }
  }

  std::vector<std::thread> th_;
  Job jobs_[2];
  std::atomic<uint64_t> ctr_{0};  // generation << 32 | next chunk
  std::atomic<size_t> done_{0};
  std::atomic<uint64_t> gen_{0};
  std::atomic<int> parked_{0};
  std::atomic<bool> stop_{false};
  std::mutex mu_;
  std::condition_variable cv_;
};

// copy threads for a process allowed `cpus` CPUs: three quarters of them,
// 1..12 (on a 16-CPU share, 12 threads and the caller fill the 4.28 MB of
// a C2 request 11 us sooner than 8 do; 16 gain nothing more)
inline int copy_threads() {
  cpu_set_t set;
  int cpus = 8;
  if (sched_getaffinity(0, sizeof set, &set) == 0) cpus = CPU_COUNT(&set);
  const int n = cpus * 3 / 4;
  return n < 1 ? 1 : n > 12 ? 12 : n;
}

}  // namespace tk
