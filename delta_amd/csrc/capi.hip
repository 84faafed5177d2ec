// Error reporting and ABI version for the delta_hip C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "delta_common.h"

namespace delta {

static thread_local char g_error[512] = {0};

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = 0; }

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(DELTA_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return DELTA_OK;
}

}  // namespace delta

extern "C" DELTA_EXPORT const char *delta_last_error(void) { return delta::g_error; }

extern "C" DELTA_EXPORT int delta_abi_version(void) { return 202; }
