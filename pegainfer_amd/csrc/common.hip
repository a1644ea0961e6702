// Host-side helpers shared by every entry point: thread-local last error,
// launch-status mapping, cached compute-unit counts.
#include "common.h"

#include <stdarg.h>
#include <stdio.h>

#include <atomic>

namespace pega {
namespace {
thread_local char g_last_error[512] = "";
// per-device CU counts, filled on first use by whichever thread gets there
std::atomic<int> g_cu_count[64];
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t err = hipPeekAtLastError();
  if (err == hipSuccess) return kSuccess;
  (void)hipGetLastError();  // clear the sticky launch error
  return fail(kLaunchFailed, "%s: launch failed: %s", what, hipGetErrorString(err));
}

int current_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int cached = g_cu_count[dev].load(std::memory_order_relaxed);
    if (cached > 0) return cached;
  }
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  if (dev < 64) g_cu_count[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

}  // namespace pega

// Reason for the last non-zero status returned on this thread (never NULL).
PEGA_API const char* pegainfer_kernels_last_error() { return pega::g_last_error; }
