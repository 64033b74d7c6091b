#include "status.hpp"

#include <stdarg.h>
#include <stdio.h>

namespace dsa {

namespace {
thread_local char g_message[512] = "";
}

int fail(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_message, sizeof(g_message), fmt, args);
  va_end(args);
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return DSA_STATUS_OK;
  return fail(DSA_STATUS_HIP_ERROR, "%s: %s", what, hipGetErrorString(err));
}

int check_launch(const char* what) { return check_hip(hipGetLastError(), what); }

}  // namespace dsa

extern "C" const char* dsa_last_error(void) { return dsa::g_message; }

extern "C" int dsa_abi_version(void) { return DSA_ABI_VERSION; }
