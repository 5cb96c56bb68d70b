// Error reporting for the C ABI: a per-thread message buffer and HIP launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "fw_common.h"

namespace {
thread_local char g_error[512] = "";
}

int fw_fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int fw_check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fw_fail(FW_EHIP, "%s: %s", what, hipGetErrorString(err));
  return FW_OK;
}

extern "C" const char* fw_last_error(void) { return g_error; }

extern "C" int fw_version(void) { return 1; }
