// Host-side plumbing shared by every entry point: version, thread-local error
// text, launch-status checks.
#include <cstdarg>
#include <cstdio>

#include "smaq_common.h"

namespace smaq {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
    return SMAQ_ELAUNCH;
  }
  return SMAQ_OK;
}

}  // namespace smaq

extern "C" int smaq_version(void) { return 100; }

extern "C" const char* smaq_last_error(void) { return smaq::g_last_error; }
