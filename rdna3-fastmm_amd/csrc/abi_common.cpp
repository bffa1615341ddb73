// Error channel and library identity of the C ABI.
#include "abi_common.h"

#include <atomic>
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

// Compute units of the current device (cached per device; 0 if unknown).
int compute_units() {
  static std::atomic<int> cached[64];  // zero-initialized
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return 0;
  int units = cached[device].load(std::memory_order_relaxed);
  if (units == 0) {
    if (hipDeviceGetAttribute(&units, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    cached[device].store(units, std::memory_order_relaxed);
  }
  return units;
}

}  // namespace fastmm

extern "C" int fastmm_abi_version(void) { return FASTMM_ABI_VERSION; }

extern "C" const char* fastmm_last_error(void) { return fastmm::last_error; }
