// C-ABI plumbing shared by every entry point: the per-thread last-error message and launch checks.
#include "rh3_common.hpp"

namespace rh3 {

namespace {
thread_local std::string g_error;
}

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

void clear_error() { g_error.clear(); }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return RH3_ELAUNCH;
  }
  return RH3_OK;
}

int device_cus() {
  static int cached[64] = {0};  // per device; a race only repeats the same query
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev] = n;
  return n;
}

}  // namespace rh3

extern "C" const char* rh3_last_error(void) { return rh3::g_error.c_str(); }

extern "C" int rh3_abi_version(void) { return 3; }
