// Error channel and library identity of the C ABI.
#include "abi_common.h"

#include <stdarg.h>
#include <stdio.h>

namespace fastmm {

namespace {
thread_local char last_error[512] = "";
}

int fail(int code, const char* format, ...) {
  va_list args;
  va_start(args, format);
  vsnprintf(last_error, sizeof(last_error), format, args);
  va_end(args);
  return code;
}

int check_launch(const char* what) {
  const hipError_t status = hipGetLastError();
  if (status != hipSuccess) {
    return fail(FASTMM_ERROR_LAUNCH, "%s: %s", what, hipGetErrorString(status));
  }
  return FASTMM_OK;
}

void clear_error() { last_error[0] = '\0'; }

}  // namespace fastmm

extern "C" int fastmm_abi_version(void) { return FASTMM_ABI_VERSION; }

extern "C" const char* fastmm_last_error(void) { return fastmm::last_error; }
