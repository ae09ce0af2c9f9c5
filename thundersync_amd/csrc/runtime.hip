// Library identity, error reporting and device attributes.
#include "common.h"
#include "../../include/thundersync_hip.h"

namespace ts {

static thread_local char g_error[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return TS_ERR_LAUNCH;
  }
  return TS_OK;
}

}  // namespace ts

extern "C" {

const char* ts_hip_version(void) { return "thundersync_hip 0.1.0 gfx950"; }

const char* ts_hip_last_error(void) { return ts::g_error; }

int ts_device_clocks(int device, int* cus, int* clock_khz, int* mem_clock_khz, int* mem_bus_bits) {
  TS_CHECK_ARG(cus && clock_khz && mem_clock_khz && mem_bus_bits, "ts_device_clocks: null pointer");
  const struct {
    hipDeviceAttribute_t attr;
    int* out;
  } want[] = {{hipDeviceAttributeMultiprocessorCount, cus},
              {hipDeviceAttributeClockRate, clock_khz},
              {hipDeviceAttributeMemoryClockRate, mem_clock_khz},
              {hipDeviceAttributeMemoryBusWidth, mem_bus_bits}};
  for (const auto& w : want) {
    if (hipDeviceGetAttribute(w.out, w.attr, device) != hipSuccess) {
      ts::set_error("ts_device_clocks: hipDeviceGetAttribute failed on device %d", device);
      return TS_ERR_LAUNCH;
    }
  }
  return TS_OK;
}

}  // extern "C"
