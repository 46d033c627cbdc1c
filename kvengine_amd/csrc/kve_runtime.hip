// Error reporting and version information for the C ABI.

#include <cstdarg>

#include "kve_common.h"

namespace kve {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return KVE_ELAUNCH;
  }
  return KVE_OK;
}

}  // namespace kve

extern "C" const char* kve_last_error(void) { return kve::g_err; }

extern "C" const char* kve_version(void) { return "kve 0.1 gfx950"; }
