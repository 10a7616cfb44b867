// Error reporting shared by every entry point: a thread-local message and HIP launch checks.
#include <stdarg.h>
#include <stdio.h>

#include "lsk_common.h"

namespace {
thread_local char g_err[512] = "";
}

namespace lsk {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return LSK_ERR_HIP;
  }
  return LSK_OK;
}

}  // namespace lsk

extern "C" const char* lsk_last_error(void) { return g_err; }

extern "C" const char* lsk_version(void) { return "lockstep_amd 0.1 (gfx950)"; }
