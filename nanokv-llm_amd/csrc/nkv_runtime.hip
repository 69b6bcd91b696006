// Error reporting and version entry points of the C ABI.
#include "nkv_common.h"

#include <string.h>

namespace nkv {

static thread_local char g_last_error[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return NKV_ELAUNCH;
  }
  return NKV_OK;
}

}  // namespace nkv

extern "C" const char* nkv_last_error(void) { return nkv::g_last_error; }

extern "C" const char* nkv_version(void) { return "nkv-amd 0.1.0 gfx950"; }
