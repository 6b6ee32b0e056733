// Host-side error reporting shared by every entry point.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

namespace trida {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TRIDA_ERR_LAUNCH;
  }
  return TRIDA_OK;
}

}  // namespace trida

extern "C" int trida_version(void) { return 100; }
extern "C" const char* trida_last_error(void) { return trida::g_err; }
