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

// Readers of the debug words of every source file (debug build), registered while the
// library loads.
static int (*g_debug_takers[16])(uint32_t*, int);
static int g_debug_n = 0;
static bool g_debug_overflow = false;

bool debug_register(int (*take)(uint32_t*, int)) {
  if (g_debug_n < 16) g_debug_takers[g_debug_n++] = take;
  else g_debug_overflow = true;
  return true;
}

}  // namespace nkv

extern "C" const char* nkv_last_error(void) { return nkv::g_last_error; }

extern "C" int nkv_debug_flags(uint32_t* flags, int clear) {
  NKV_REQUIRE(flags, NKV_EINVAL, "debug_flags: null pointer");
  *flags = 0;
#ifdef NKV_DEBUG
  NKV_REQUIRE(!nkv::g_debug_overflow, NKV_EUNSUPPORTED, "debug_flags: too many source files");
  const hipError_t e = hipDeviceSynchronize();
  NKV_REQUIRE(e == hipSuccess, NKV_ELAUNCH, "debug_flags: %s", hipGetErrorString(e));
  for (int i = 0; i < nkv::g_debug_n; ++i) {
    const int rc = nkv::g_debug_takers[i](flags, clear);
    NKV_REQUIRE(rc == NKV_OK, rc, "debug_flags: reading a debug word failed");
  }
  return NKV_OK;
#else
  (void)clear;
  nkv::set_error("debug_flags: built without NKV_DEBUG (use libnkv_amd_debug.so)");
  return NKV_EUNSUPPORTED;
#endif
}

extern "C" const char* nkv_version(void) { return "nkv-amd 0.1.0 gfx950"; }
