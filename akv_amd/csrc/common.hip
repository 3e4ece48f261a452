// Error state and version of the akv_amd C ABI.
#include <string>

#include "common.h"

namespace akv {

std::string& last_error() {
  static thread_local std::string message;
  return message;
}

int fail(int code, const char* fmt, ...) {
  // sized to the message: some list every offending index
  va_list ap, again;
  va_start(ap, fmt);
  va_copy(again, ap);
  const int len = vsnprintf(nullptr, 0, fmt, ap);
  va_end(ap);
  std::string msg(len > 0 ? static_cast<size_t>(len) : 0, '\0');
  if (len > 0) vsnprintf(&msg[0], msg.size() + 1, fmt, again);
  va_end(again);
  last_error() = std::move(msg);
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
