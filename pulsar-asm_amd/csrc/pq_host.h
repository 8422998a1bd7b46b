// pq_host.h -- host-side helpers of the C ABI: error state and argument checks.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "../../include/pulsar_amd.h"

namespace pq {

// Records the message of the calling thread's last failure and returns code.
int fail(int code, const char *fmt, ...);

inline bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// An integer launch-shape override from the environment (0 when unset); read
// once per call site into a function-local static (thread-safe initialization).
inline int env_int(const char *name) {
  const char *e = getenv(name);
  return e ? atoi(e) : 0;
}

// Checks the launch that was just queued; a failed launch returns
// PQ_ERR_LAUNCH and produces no output (the reference's rule: no number from
// a kernel that did not run, lfm3_nanode.cu:4957-4961).
inline int check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PQ_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PQ_OK;
}

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Timing hook (pq_time_next_launch): events that the next kernel launch of the
// calling thread carries on its own dispatch packet.
struct TimedLaunch {
  hipEvent_t start = nullptr, stop = nullptr;
};
TimedLaunch &timed_launch();

// Launches a kernel; if pq_time_next_launch armed a pair of events, they are
// attached to this dispatch (hipExtLaunchKernelGGL) and the pair is consumed.
template <typename... Args, typename F>
inline void launch(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
  TimedLaunch &t = timed_launch();
  if (t.start != nullptr) {
    hipEvent_t a = t.start, b = t.stop;
    t.start = t.stop = nullptr;
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, st, a, b, 0, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
  }
}

}  // namespace pq

#define PQ_REQUIRE(cond, code, ...) \
  do {                              \
    if (!(cond)) return ::pq::fail((code), __VA_ARGS__); \
  } while (0)
