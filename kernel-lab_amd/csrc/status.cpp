// Status strings, per-thread error detail and device queries for the C-ABI.
#include <cstdio>
#include <cstring>
#include <mutex>
#include <vector>

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
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (static_cast<size_t>(dev) >= cache.size()) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
      return 0;
    }
    cache[dev] = cus;
  }
  return cache[dev];
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
