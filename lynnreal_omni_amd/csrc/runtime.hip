// runtime.hip - ABI version, last-error state and the device-support query.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>

#include "lr_runtime.h"

namespace lr {

static thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t err, const char* where) {
  // Clear the sticky error so that the next call starts clean.
  (void)hipGetLastError();
  return fail(err == hipErrorOutOfMemory ? LR_ENOMEM : LR_EHIP, "%s: %s (hip error %d)", where,
              hipGetErrorString(err), (int)err);
}

int compute_units() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 256;
  }
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    n = 256;
  }
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace lr

extern "C" int lr_abi_version(void) { return LR_ABI_VERSION; }

extern "C" const char* lr_last_error(void) { return lr::g_last_error; }

extern "C" int lr_device_supported(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}
