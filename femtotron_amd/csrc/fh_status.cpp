// Library version and the per-thread error string behind fh_last_error().
#include <hip/hip_runtime.h>

#include <string>

#include "fh_common.hpp"

namespace fh {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return fail(FH_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  }
  return FH_OK;
}

}  // namespace fh

extern "C" int fh_abi_version(void) { return FH_ABI_VERSION; }

extern "C" const char* fh_last_error(void) { return fh::g_last_error.c_str(); }
