// runtime.cpp -- sticky error state and library identity for libubridge_hip.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace {
thread_local int g_err = UB_OK;
thread_local char g_msg[512] = {0};
}  // namespace

int ub_set_error(int code, const char* fmt, ...) {
  g_err = code;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

int ub_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return ub_set_error(UB_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return UB_OK;
}

UB_API int ubridge_last_error(void) {
  int e = g_err;
  g_err = UB_OK;
  return e;
}

UB_API const char* ubridge_last_error_string(void) { return g_msg; }

UB_API const char* ubridge_version(void) { return "ubridge_amd 0.1 gfx950"; }
