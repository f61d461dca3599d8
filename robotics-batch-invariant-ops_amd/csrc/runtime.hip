// Library state: per-thread error message and the once-per-device property cache.  Nothing else
// is mutable, so every entry point is re-entrant.
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "biops_common.h"

namespace biops {

namespace {
thread_local char g_error[512] = "";
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];  // 0 = unknown
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(BIOPS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return BIOPS_OK;
}

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  int v = g_cus[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    return -1;
  g_cus[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace biops

extern "C" const char* biops_version(void) { return "0.2.0-mi355x"; }

extern "C" const char* biops_last_error(void) { return biops::g_error; }

extern "C" int biops_compute_units(void) {
  const int n = biops::device_cus();
  if (n <= 0) biops::set_error("no HIP device");
  return n;
}
