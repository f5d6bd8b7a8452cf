// Error state and version entry points of the C ABI.
#include <cstdarg>
#include <cstdio>

#include "sage_common.h"

namespace sage {

namespace {
thread_local char g_last_error[512] = {0};
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(SAGE_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return SAGE_OK;
}

}  // namespace sage

extern "C" int sage_abi_version(void) { return SAGE_ABI_VERSION; }

extern "C" const char* sage_last_error(void) { return sage::g_last_error; }
