// Host-side helpers of libart_moe: error reporting and device properties.
#include <stdarg.h>

#include <mutex>

#include "common.h"

namespace art {

static thread_local std::string g_last_error;

void set_error(const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int check_launch(const char *what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: HIP launch failed: %s", what, hipGetErrorString(err));
    return ART_MOE_ERR_HIP;
  }
  return ART_MOE_OK;
}

// Compute-unit count of the current device, cached per device id.
int device_cu_count() {
  static std::mutex mu;
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

}  // namespace art

extern "C" int art_moe_version(void) { return 100; }

extern "C" const char *art_moe_last_error(void) { return art::g_last_error.c_str(); }
