// Host-side status plumbing of the C ABI: a per-thread last-error message, version string.
#include <stdarg.h>
#include <stdio.h>

#include "dspark_common.h"

namespace dspark {

static thread_local char g_last_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(DSPARK_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return DSPARK_OK;
}

}  // namespace dspark

extern "C" const char* dspark_last_error(void) { return dspark::g_last_error; }

extern "C" const char* dspark_version(void) { return "dspark-rocm 0.1.0 (gfx950)"; }
