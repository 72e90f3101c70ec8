// Host-side helpers shared by the C-ABI entry points: error state, launch checks, device properties.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/rk_path.h"

namespace rk {

// Record an error message for rk_last_error() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Check hipGetLastError() after a launch; returns RK_OK or RK_ERR_HIP with the message recorded.
int check_launch(const char* what);

// Compute units of the current device (cached per device id).
int device_cus();

// Raise the dynamic LDS limit of kernel `func` to `bytes` on the current device (once per device, kernel and size).
int allow_dynamic_lds(const void* func, size_t bytes);

inline size_t ceil_div(size_t a, size_t b) { return (a + b - 1) / b; }

}  // namespace rk
