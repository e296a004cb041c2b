// Host-side helpers shared by the C-ABI entry points: status codes, the
// thread-local last-error message, and argument checks. No C++ exception ever
// crosses the ABI: every entry point returns a PF_* status.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/pairformer_hip.h"

namespace pf {

void set_error(int code, const char* fmt, ...);
int ok();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Returns PF_OK or records a launch error.
int check_launch(const char* what);

inline size_t round_up(size_t x, size_t m) { return (x + m - 1) / m * m; }

// Token padding used by the pair-plane and attention buffers.
inline int pad128(int n) { return (int)round_up((size_t)n, 128); }

// Compute units of the current device (cached per device), for persistent grids.
int cu_count();

// Opt-in per-kernel timing (pf_kernel_timer_*). Construct before a launch site and call
// stop() after it: both record a HIP event on the launch stream (without the system-scope
// fence, so no cache flush), and the site's time is the difference of the two events' end
// timestamps, each read against one reference event recorded when timing starts. Measured on
// gfx950: an event's start timestamp can come before the work queued ahead of it has ended
// (back-to-back 52 us kernels read 100-110 us from start to end), its end timestamp cannot;
// end to end, the figures exceed the rocprofv3 kernel trace of the same launches by the
// ~5 us of the two events. Both are no-ops unless the site's name is the one selected with
// pf_kernel_timer_start.
class KernelTimer {
 public:
  KernelTimer(const char* name, hipStream_t stream);
  void stop();

 private:
  hipStream_t stream_;
  void* start_ = nullptr;
};

}  // namespace pf

#define PF_REQUIRE(cond, code, ...)          \
  do {                                       \
    if (!(cond)) {                           \
      pf::set_error((code), __VA_ARGS__);    \
      return (code);                         \
    }                                        \
  } while (0)
