// Library-wide C-ABI helpers: last-error string and runtime identification.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"
#include "../../include/tritium_hip.h"

namespace {
thread_local char g_last_error[1024] = "";
}

namespace tri {

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(TRI_ELAUNCH, "%s: %s", what, hipGetErrorString(err));
  }
  return TRI_OK;
}

}  // namespace tri

extern "C" const char* tritium_last_error(void) { return g_last_error; }

extern "C" int tritium_abi_version(void) { return TRITIUM_HIP_ABI_VERSION; }

extern "C" int tritium_runtime_version(void) {
  int v = 0;
  if (hipRuntimeGetVersion(&v) != hipSuccess) return -1;
  return v;
}
