// Error state and device queries shared by the entry points.
#include "li_common.h"

#include <mutex>
#include <string>
#include <vector>

namespace li {

namespace {
thread_local std::string g_last_error;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(LI_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return LI_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> counts;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if ((int)counts.size() <= dev) counts.resize(dev + 1, 0);
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

}  // namespace li

extern "C" const char* li_last_error_string(void) { return li::g_last_error.c_str(); }

extern "C" int li_abi_version(void) { return 7; }

// Digest of the sources and flags this library was built from, passed in by
// the build script; the Python loader refuses a library whose digest differs
// from the sources beside it.
#ifndef LI_BUILD_ID
#define LI_BUILD_ID "unknown"
#endif
extern "C" const char* li_build_id(void) { return LI_BUILD_ID; }
