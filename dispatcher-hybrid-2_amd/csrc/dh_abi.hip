// ABI bookkeeping: version and the thread-local last-error message.
#include <stdarg.h>
#include <stdio.h>

#include "dh_common.h"

static thread_local char g_last_error[512] = "";

int dh_fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int dh_check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return dh_fail(DH_ERR_LAUNCH_FAILED, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return DH_OK;
}

extern "C" int dh_abi_version(void) { return DH_ABI_VERSION; }

extern "C" const char* dh_last_error(void) { return g_last_error; }
