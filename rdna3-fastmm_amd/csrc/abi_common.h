// Host-side helpers shared by the C ABI entry points.
#ifndef FASTMM_ABI_COMMON_H
#define FASTMM_ABI_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fastmm_amd.h"

namespace fastmm {

// Record a printf-style message for fastmm_last_error() and return `code`.
int fail(int code, const char* format, ...) __attribute__((format(printf, 2, 3)));

// FASTMM_OK, or FASTMM_ERROR_LAUNCH with the HIP error text after a launch.
int check_launch(const char* what);

// Clear the thread's last error at the start of an entry point.
void clear_error();

// Compute units of the current device (cached per device; 0 if unknown).
int compute_units();

inline bool aligned_to(const void* pointer, uintptr_t bytes) {
  return (reinterpret_cast<uintptr_t>(pointer) % bytes) == 0;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace fastmm

#endif  // FASTMM_ABI_COMMON_H
