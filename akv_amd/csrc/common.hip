// Error state and version of the akv_amd C ABI.
#include "common.h"

namespace akv {

std::string& last_error() {
  static thread_local std::string message;
  return message;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess)
    return fail(AKV_EHIP, "%s: HIP launch failed: %s", what, hipGetErrorString(err));
  return AKV_OK;
}

}  // namespace akv

extern "C" const char* akv_last_error(void) { return akv::last_error().c_str(); }

extern "C" const char* akv_version(void) { return "akv_amd 0.1.0 gfx950"; }
