// profiler.h -- adds the elapsed wall time of a scope to a sink in ms
// (reference include/dsd/profiler.h:7-27).
#pragma once

#include <chrono>

namespace dsd {

class ScopedStageTimer {
 public:
  explicit ScopedStageTimer(double* sink_ms) : sink_ms_(sink_ms), start_(Clock::now()) {}
  ~ScopedStageTimer() {
    if (sink_ms_ != nullptr) {
      *sink_ms_ += std::chrono::duration<double, std::milli>(Clock::now() - start_).count();
    }
  }
  ScopedStageTimer(const ScopedStageTimer&) = delete;
  ScopedStageTimer& operator=(const ScopedStageTimer&) = delete;

 private:
  using Clock = std::chrono::steady_clock;
  double* sink_ms_ = nullptr;
  Clock::time_point start_;
};

}  // namespace dsd
