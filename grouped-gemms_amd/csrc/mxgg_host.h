// Host-side helpers of libmxgg: per-thread error state and launch checks.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mxgg.h"

namespace mxgg {

// Record a failure for mxgg_last_error_string() and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// hipGetLastError() after a launch, mapped to the C-ABI status convention.
int launch_status(const char* what);
// MXGG_ERR_NO_DEVICE unless the current device is gfx950.
int require_device();

}  // namespace mxgg
