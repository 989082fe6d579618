// Error reporting and version of the nvhip C ABI.
#include <cstdio>

#include "common.h"

namespace nvhip {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int invalid(const std::string& msg) {
  g_last_error = msg;
  return NVHIP_EINVAL;
}

int check_launch(const char* kernel) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    g_last_error = std::string(kernel) + ": launch failed: " + hipGetErrorString(err);
    return NVHIP_ELAUNCH;
  }
  return NVHIP_OK;
}

}  // namespace nvhip

extern "C" int nvhip_abi_version(void) { return 7; }

extern "C" const char* nvhip_last_error(void) { return nvhip::g_last_error.c_str(); }
