// Library-level C ABI: version and per-thread error reporting.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace ntops {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(NTOPS_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return NTOPS_OK;
}

}  // namespace ntops

extern "C" int ntops_abi_version(void) { return 1; }

extern "C" const char* ntops_last_error(void) { return ntops::g_last_error; }
