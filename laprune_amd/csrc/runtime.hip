// runtime.hip — error state, ABI version and per-device facts of the C ABI.
#include "common.h"

#include <mutex>

namespace lap {

namespace {
thread_local std::string t_error;

constexpr int kMaxDevices = 64;
DevInfo g_dev[kMaxDevices];
std::once_flag g_dev_once[kMaxDevices];
int g_dev_status[kMaxDevices];
}  // namespace

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  t_error = buf;
}

void clear_error() { t_error.clear(); }

int device_info(DevInfo* out) {
  int dev = 0;
  LAP_HIP(hipGetDevice(&dev), "hipGetDevice");
  LAP_CHECK_CODE(dev >= 0 && dev < kMaxDevices, LAP_ERR_UNSUPPORTED,
                 "device ordinal %d exceeds the supported %d devices", dev, kMaxDevices);
  std::call_once(g_dev_once[dev], [dev]() {
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) {
      g_dev_status[dev] = LAP_ERR_HIP;
      return;
    }
    g_dev[dev].cu_count = p.multiProcessorCount;
    g_dev[dev].lds_per_block = (int)p.sharedMemPerBlock;
    g_dev[dev].wave_size = p.warpSize;
    g_dev_status[dev] = LAP_OK;
  });
  if (g_dev_status[dev] != LAP_OK) {
    set_error("hipGetDeviceProperties failed for device %d", dev);
    return g_dev_status[dev];
  }
  *out = g_dev[dev];
  return LAP_OK;
}

}  // namespace lap

extern "C" {

const char* lap_last_error(void) { return lap::t_error.c_str(); }

int lap_abi_version(void) { return 7; }

int lap_device_info(int* cu_count, int* lds_bytes_per_block, int* wave_size) {
  lap::DevInfo d;
  int st = lap::device_info(&d);
  if (st != LAP_OK) return st;
  if (cu_count) *cu_count = d.cu_count;
  if (lds_bytes_per_block) *lds_bytes_per_block = d.lds_per_block;
  if (wave_size) *wave_size = d.wave_size;
  return LAP_OK;
}

}  // extern "C"
