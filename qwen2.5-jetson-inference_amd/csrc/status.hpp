// Error plumbing for the C ABI: entry points never throw; they return an
// infer_hip_status and leave a message for infer_hip_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include "infer_linear.h"

namespace qlin {

// Record `message` as this thread's last error and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clear the last error and return INFER_HIP_OK.
int ok();

// Map the launch status of the most recent kernel to a status code.
int check_launch(const char* what);

}  // namespace qlin
