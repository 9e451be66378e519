// Library-wide C ABI helpers: version, per-thread error message, device check.
#include <cstring>

#include "common.hpp"

namespace ta {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return TA_ERR_LAUNCH;
  }
  return TA_OK;
}

static int device_attribute(hipDeviceAttribute_t attr, int (&cache)[64]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (cache[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, attr, dev) != hipSuccess || n <= 0) return 0;
    cache[dev] = n;
  }
  return cache[dev];
}

int device_cus() {
  static int cache[64] = {0};
  return device_attribute(hipDeviceAttributeMultiprocessorCount, cache);
}

int device_lds_per_cu() {
  static int cache[64] = {0};
  return device_attribute(hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, cache);
}

}  // namespace ta

extern "C" int ta_abi_version(void) { return TA_ABI_VERSION; }

extern "C" const char* ta_last_error(void) { return ta::g_last_error.c_str(); }

extern "C" int ta_device_supported(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}
