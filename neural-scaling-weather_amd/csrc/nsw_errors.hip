// Thread-local error reporting of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "nsw_common.h"

namespace nsw {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(NSW_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return NSW_OK;
}

}  // namespace nsw

extern "C" const char* nsw_last_error(void) { return nsw::g_last_error; }

extern "C" int nsw_version(void) { return 1; }
