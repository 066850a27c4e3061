// CPU stress of the copy threads' pool (toktier_amd/csrc/tk_copy_pool.h),
// built by tests/test_copy_pool.py, with ThreadSanitizer and without. Many
// back-to-back jobs of varying sizes, some after a pause long enough for
// the workers to sleep: every chunk of every job must run exactly once, and
// only under its own job's function (a worker that wakes late must not take
// a chunk of a later job with an earlier job's function).
#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

#include "../toktier_amd/csrc/tk_copy_pool.h"

int main(int argc, char** argv) {
  const int threads = argc > 1 ? std::atoi(argv[1]) : 4;
  const int jobs = argc > 2 ? std::atoi(argv[2]) : 20000;
  tk::CopyPool pool(threads);
  std::vector<std::atomic<int>> hits(512);
  std::atomic<int> current{-1};
  long bad = 0;
  for (int j = 0; j < jobs; ++j) {
    const size_t n = 1 + (size_t)((uint32_t)j * 2654435761u >> 7) % 300;
    for (size_t k = 0; k < n; ++k) hits[k].store(0, std::memory_order_relaxed);
    std::atomic<int> wrong{0};
    current.store(j);
    pool.run(n, [&, j](size_t k) {
      if (current.load() != j || k >= n) {
        wrong.fetch_add(1);
        return;
      }
      hits[k].fetch_add(1, std::memory_order_relaxed);
    });
    current.store(-1);
    for (size_t k = 0; k < n; ++k)
      if (hits[k].load() != 1) ++bad;
    bad += wrong.load();
    if (j % 4000 == 3999)  // long enough for the workers to go to sleep
      std::this_thread::sleep_for(tk::CopyPool::SPIN * 3);
  }
  std::printf("%s: %d threads, %d jobs, %ld bad chunks\n", bad ? "FAIL" : "ok",
              threads, jobs, bad);
  return bad ? 1 : 0;
}
