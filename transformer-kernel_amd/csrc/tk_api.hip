// Library-wide entry points and error plumbing for libtkmi.
#include "tk_common.hpp"

namespace tk {

static thread_local char g_err[512] = {0};

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

void clear_error() { g_err[0] = 0; }

const char* last_error() { return g_err; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(e));
    return TK_ERR_HIP;
  }
  return TK_OK;
}

}  // namespace tk

extern "C" int tk_version(void) { return TKMI_ABI_VERSION; }

extern "C" const char* tk_last_error_string(void) { return tk::last_error(); }
