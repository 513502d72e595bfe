// Host-side helpers shared by the C-ABI entry points: status reporting with a
// per-thread detail string, and the device compute-unit count.
#pragma once

#include <hip/hip_runtime.h>

#include "kernel_lab.h"

namespace kl {

// Records `detail` as the calling thread's last error and returns `status`.
int fail(int status, const char* detail);

// Records a HIP error (its name and text) and returns KL_ERR_HIP.
int fail_hip(hipError_t err, const char* what);

// Clears the calling thread's last error and returns KL_OK.
int ok();

// Returns the status of the most recent launch on this thread.
int check_launch(const char* what);

// Compute units of the current device (cached per device), or 0 on error.
int current_cu_count();

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace kl
