// Status strings, per-thread error detail and device queries for the C-ABI.
#include <atomic>
#include <cstdio>
#include <cstring>

#include "kl_internal.h"

namespace kl {
namespace {

thread_local char g_last_error[512] = "";

}  // namespace

int fail(int status, const char* detail) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s", detail ? detail : "");
  return status;
}

int fail_hip(hipError_t err, const char* what) {
  std::snprintf(g_last_error, sizeof(g_last_error), "%s: %s (%s)", what, hipGetErrorName(err),
                hipGetErrorString(err));
  return KL_ERR_HIP;
}

int ok() {
  g_last_error[0] = '\0';
  return KL_OK;
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) return fail_hip(err, what);
  return ok();
}

int current_cu_count() {
  // One slot per device, filled on first use; a racing second fill stores the
  // same value, so no lock is needed.
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev >= kMaxDevices) {
    int cus = 0;
    return hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? cus : 0;
  }
  int cus = cache[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev].store(cus, std::memory_order_relaxed);
  }
  return cus;
}

}  // namespace kl

extern "C" {

const char* kl_status_string(int status) {
  switch (status) {
    case KL_OK:
      return "success";
    case KL_ERR_INVALID_ARGUMENT:
      return "invalid argument";
    case KL_ERR_UNSUPPORTED:
      return "unsupported shape or dtype";
    case KL_ERR_WORKSPACE:
      return "workspace missing or too small";
    case KL_ERR_HIP:
      return "HIP runtime error";
    default:
      return "unknown status";
  }
}

const char* kl_last_error(void) { return kl::g_last_error; }

int kl_version(void) { return 100; }

}  // extern "C"
