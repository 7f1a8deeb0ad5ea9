// Library-level C ABI: version and per-thread error reporting.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "common.h"

namespace ntops {

static thread_local char g_last_error[512] = "";
static thread_local char g_last_kernel[128] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void note_kernel(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_kernel, sizeof(g_last_kernel), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(NTOPS_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return NTOPS_OK;
}

int cu_count_cached() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace ntops

extern "C" int ntops_abi_version(void) { return 2; }

extern "C" const char* ntops_last_error(void) { return ntops::g_last_error; }

extern "C" const char* ntops_last_kernel(void) { return ntops::g_last_kernel; }
