// Error reporting of the C ABI (thread-local last-error message).
#include "zkv_common.hpp"

namespace zkv {

static thread_local char g_last_error[512] = "";

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

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(ZKV_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return ZKV_OK;
}

}  // namespace zkv

extern "C" const char* zkv_last_error(void) { return zkv::g_last_error; }

extern "C" const char* zkv_version(void) { return "zoomkv_gfx950 0.1 (format R, format Q v1)"; }
