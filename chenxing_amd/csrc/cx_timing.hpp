// cx_timing.hpp -- opt-in per-launch kernel timing.  While timing is on,
// every library kernel is launched with hipExtLaunchKernelGGL and a start /
// stop event pair that the dispatch itself records (the kernel's own
// execution interval on its stream, not the host's launch overhead).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stdint.h>
#include <mutex>
#include <vector>

#include "cx_sampler.h"

namespace cx {

struct TimedLaunch {
  hipEvent_t a, b;
};

struct Timing {
  bool on = false;
  std::mutex mu;
  std::vector<TimedLaunch> rec[CX_KERNEL_KINDS];
  std::vector<hipEvent_t> pool;

  hipEvent_t take() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
  }
};

Timing& timing();

// Launch `kernel`; with timing on, its execution interval is recorded under
// `kind` (one of the CX_KERNEL_* ids).
template <typename F, typename... Args>
inline void timed_launch(int kind, F kernel, dim3 grid, dim3 block, uint32_t lds, hipStream_t s,
                         Args... args) {
  Timing& T = timing();
  if (T.on) {
    hipEvent_t a = nullptr, b = nullptr;
    {
      std::lock_guard<std::mutex> g(T.mu);
      a = T.take();
      b = T.take();
    }
    if (a && b) {
      hipExtLaunchKernelGGL(kernel, grid, block, lds, s, a, b, 0u, args...);
      std::lock_guard<std::mutex> g(T.mu);
      T.rec[kind].push_back({a, b});
      return;
    }
  }
  hipLaunchKernelGGL(kernel, grid, block, lds, s, args...);
}

}  // namespace cx
