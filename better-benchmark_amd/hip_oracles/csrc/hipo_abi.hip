// ABI bookkeeping: version, per-thread error message, device-property cache.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "hipo_common.h"

namespace hipo {

namespace {
thread_local char g_error[512] = {0};

constexpr int kMaxDevices = 64;
DeviceInfo g_devices[kMaxDevices];
std::once_flag g_device_once[kMaxDevices];
}  // namespace

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_error[0] = 0; }

const DeviceInfo* device_info() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    return nullptr;
  }
  std::call_once(g_device_once[dev], [dev]() {
    hipDeviceProp_t prop;
    DeviceInfo info{dev, 0, 0, 0};
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      info.cu_count = prop.multiProcessorCount;
      info.max_threads_per_cu = prop.maxThreadsPerMultiProcessor;
      info.lds_per_block = prop.sharedMemPerBlock;
    }
    g_devices[dev] = info;
  });
  return g_devices[dev].cu_count > 0 ? &g_devices[dev] : nullptr;
}

int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(err));
    return static_cast<int>(err);
  }
  return 0;
}

}  // namespace hipo

extern "C" int hipo_abi_version(void) { return HIPO_ABI_VERSION; }

extern "C" const char* hipo_last_error(void) { return hipo::g_error; }
