// Status codes and the thread-local last-error message of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.hpp"

namespace {
thread_local char g_last_error[512] = "";
}

namespace fmoe_host {

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(FMOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return FMOE_OK;
}

}  // namespace fmoe_host

extern "C" {

const char* fmoe_status_string(int status) {
  switch (status) {
    case FMOE_OK: return "ok";
    case FMOE_ERR_INVALID: return "invalid argument";
    case FMOE_ERR_UNSUPPORTED: return "not supported";
    case FMOE_ERR_WORKSPACE: return "workspace too small";
    case FMOE_ERR_HIP: return "HIP error";
    default: return "unknown status";
  }
}

const char* fmoe_last_error(void) { return g_last_error; }

int fmoe_abi_version(void) { return 2; }

}  // extern "C"
