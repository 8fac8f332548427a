// Error state and version entry points of the C ABI.
#include "mi_common.h"

namespace mi {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

void clear_error() { g_last_error.clear(); }

int32_t fail(int32_t status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int32_t check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(MI_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
  }
  return MI_OK;
}

}  // namespace mi

extern "C" const char* mi_last_error(void) { return mi::g_last_error.c_str(); }

extern "C" int32_t mi_abi_version(void) { return 102; }
