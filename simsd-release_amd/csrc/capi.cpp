// C-ABI housekeeping: thread-local error string, launch checks, version.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "simsd_kernels.h"

namespace simsd {

namespace {
thread_local char g_err[512] = {0};
}

int set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return -1;
}

// Non-blocking: reports launch-configuration errors without synchronising.
int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error("%s: launch failed: %s", what, hipGetErrorString(e));
  return 0;
}

}  // namespace simsd

extern "C" const char* simsd_last_error_string(void) { return simsd::g_err; }

extern "C" int simsd_abi_version(void) { return SIMSD_ABI_VERSION; }
