// Host-only helpers of the akv_amd C ABI (error reporting).
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/akv_amd.h"

namespace akv {

// Last error message of the calling host thread (akv_last_error()).
std::string& last_error();

// Records a formatted message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace akv
