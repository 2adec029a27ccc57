// bi_abi.hip — library-wide C-ABI pieces: version, thread-local error text,
// launch-status plumbing.
#include <stdarg.h>
#include <stdio.h>

#include "bi_common.h"

namespace {
thread_local char g_last_error[512] = "";
}

namespace bi_host {

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return BI_OK;
}

}  // namespace bi_host

extern "C" int bi_abi_version(void) { return BI_ABI_VERSION; }
extern "C" const char* bi_last_error(void) { return g_last_error; }
