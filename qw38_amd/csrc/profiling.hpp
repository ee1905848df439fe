// Opt-in roctx ranges around the host operations (the reference's
// src/runtime/profiling.hpp:11-36 NVTX ranges, same "qw38:op name=..." strings,
// so a rocprofv3 --marker-trace attributes kernels to operations).
// Profiling is off unless qw38_set_profiling(1) was called on the thread or
// QW38_PROFILE=1 is set in the environment.
#pragma once

#include <rocprofiler-sdk-roctx/roctx.h>

#include <cstdio>
#include <cstdlib>

namespace qw38hip::profiling {

inline bool env_enabled() {
  static const bool on = [] {
    const char* e = std::getenv("QW38_PROFILE");
    return e && std::atoi(e) != 0;
  }();
  return on;
}
inline thread_local bool enabled = false;

class ScopedRange {
 public:
  explicit ScopedRange(const char* name) noexcept : active_(enabled || env_enabled()) {
    if (active_) roctxRangePushA(name);
  }
  template <class... Args>
  ScopedRange(const char* format, Args... args) noexcept : active_(enabled || env_enabled()) {
    if (active_) {
      char name[384];
      std::snprintf(name, sizeof(name), format, args...);
      roctxRangePushA(name);
    }
  }
  ~ScopedRange() { close(); }
  void close() noexcept {
    if (active_) roctxRangePop();
    active_ = false;
  }
  ScopedRange(const ScopedRange&) = delete;
  ScopedRange& operator=(const ScopedRange&) = delete;

 private:
  bool active_;
};

}  // namespace qw38hip::profiling
