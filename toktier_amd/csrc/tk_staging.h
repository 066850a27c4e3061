// tk_staging.h -- host side of the host-to-host entry points: pinned
// staging buffers and a small pool of copy threads (internal to
// libtoktier_hip).
//
// The reference's fused lane stages the request the same way (the UTF-8
// bytes copied into a pinned buffer, then a non-blocking host-to-device
// copy; src/toktier/engine/gpu/encoder.py:462-467, :566-567). Here the copy
// into the staging is spread over several threads and followed by ONE
// transfer: on MI355X a DMA split into chunks runs at half the rate of a
// single one (each transfer command carries a fixed cost of about 10 us),
// while the copy threads fill the 4.28 MB of a C2 request at about 130
// GB/s, a third of the transfer's time. Ids come back
// without a transfer command: the compaction kernel writes them straight
// into page-locked host memory (the caller's buffer or the out staging).
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "tk_copy_pool.h"

namespace tk {

// Pinned host memory (hipHostMalloc), grown on demand.
// `dev` is its address in the device's view, for kernels that write it.
struct PinnedBuf {
  uint8_t* p = nullptr;
  uint8_t* dev = nullptr;
  size_t n = 0;
  ~PinnedBuf() { reset(); }
  void reset() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    dev = nullptr;
    n = 0;
  }
  hipError_t ensure(size_t bytes) {
    if (bytes <= n) return hipSuccess;
    reset();
    void* q = nullptr;
    hipError_t e = hipHostMalloc(&q, bytes, hipHostMallocDefault);
    if (e != hipSuccess) return e;
    void* d = nullptr;
    e = hipHostGetDevicePointer(&d, q, 0);
    if (e != hipSuccess) {
      (void)hipHostFree(q);
      return e;
    }
    p = static_cast<uint8_t*>(q);
    dev = static_cast<uint8_t*>(d);
    n = bytes;
    return hipSuccess;
  }
};

}  // namespace tk
