// lr_runtime.h - host-side helpers of the C ABI: status codes, the
// thread-local last-error message and argument checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lynnreal_amd.h"

namespace lr {

// Records `msg` (printf-style) as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Maps a HIP error to an LR status, recording hipGetErrorString.
int hip_fail(hipError_t err, const char* where);

// Checks hipGetLastError() after a launch.
inline int check_launch(const char* where) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, where);
  return LR_OK;
}

// Compute units of the current device (cached per device; 256 if the query fails).
int compute_units();

inline bool aligned(const void* p, uintptr_t bytes) { return ((uintptr_t)p % bytes) == 0; }

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace lr

#define LR_REQUIRE(cond, ...)                               \
  do {                                                      \
    if (!(cond)) return ::lr::fail(LR_EINVAL, __VA_ARGS__); \
  } while (0)
