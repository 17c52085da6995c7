// Thread-local error string behind kf_last_error() and the shared launch check.
#include <stdarg.h>
#include <stdio.h>

#include "kf_host.hpp"

namespace {
thread_local char g_err[1024] = "";
}

namespace kf {

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(KF_ELAUNCH, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  }
  return KF_OK;
}

}  // namespace kf

extern "C" const char* kf_last_error(void) { return g_err; }

extern "C" int kf_abi_version(void) { return KF_ABI_VERSION; }
