// C-ABI bookkeeping: thread-local error message and launch checking.
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/strata_hip.h"

namespace strata {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(STRATA_HIP_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
  return STRATA_HIP_OK;
}

}  // namespace strata

extern "C" const char* strata_hip_last_error(void) { return strata::g_last_error.c_str(); }

extern "C" int strata_hip_abi_version(void) { return STRATA_HIP_ABI_VERSION; }
