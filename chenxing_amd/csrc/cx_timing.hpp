// cx_timing.hpp -- opt-in hipEvent timing around library kernel launches.
#pragma once
#include <hip/hip_runtime.h>
#include <mutex>
#include <vector>

namespace cx {

struct TimedLaunch {
  hipEvent_t a, b;
};

struct Timing {
  bool on = false;
  std::mutex mu;
  std::vector<TimedLaunch> rec[5];
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

// Brackets one kernel launch with events on its stream when timing is on.
struct TimedScope {
  int kind;
  hipStream_t s;
  hipEvent_t a = nullptr, b = nullptr;
  TimedScope(int k, hipStream_t st) : kind(k), s(st) {
    Timing& T = timing();
    if (!T.on) return;
    std::lock_guard<std::mutex> g(T.mu);
    a = T.take();
    b = T.take();
    if (a) (void)hipEventRecord(a, s);
  }
  ~TimedScope() {
    if (!a || !b) return;
    (void)hipEventRecord(b, s);
    Timing& T = timing();
    std::lock_guard<std::mutex> g(T.mu);
    T.rec[kind].push_back({a, b});
  }
};

}  // namespace cx
