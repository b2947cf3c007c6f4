// Host-side error reporting and small shared utilities for libds355.
#include <cstdarg>
#include <cstdio>

#include "ds355_common.h"

namespace ds355 {

namespace {
thread_local char g_error[512] = "";
constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices] = {0};
}  // namespace

int set_error(int code, const char* fmt, ...) {
  va_list args;
  va_start(args, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, args);
  va_end(args);
  return code;
}

int clear_error() {
  g_error[0] = '\0';
  return DS_OK;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return set_error(DS_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(err));
  }
  return clear_error();
}

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  if (g_cu_count[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      cus = 256;
    }
    g_cu_count[dev] = cus;
  }
  return g_cu_count[dev];
}

}  // namespace ds355

extern "C" const char* ds_last_error(void) { return ds355::g_error; }

extern "C" int ds_abi_version(void) { return 7; }
