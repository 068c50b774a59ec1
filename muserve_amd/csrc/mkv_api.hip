// mkv_api.hip — version and per-thread error reporting of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "mkv_host.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace mkv {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* kernel) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(MKV_E_LAUNCH, "%s: launch failed: %s", kernel, hipGetErrorString(e));
  return MKV_OK;
}

}  // namespace mkv

extern "C" int mkv_version(void) { return MKV_ABI_VERSION; }

extern "C" const char* mkv_last_error(void) { return g_last_error; }
