// RMSNorm backward that allocates nothing: for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, harnesses
// that forbid hipMalloc).  It is ts_rmsnorm_bwd with its workspace -- the
// fp32 dW partial rows -- taken from `scratch`, a file-scope device array of
// TS_RMSNORM_BWD_SCRATCH_BYTES that every GPU the library runs on holds until
// the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: its
// per-device address comes from hipGetSymbolAddress, taken once per device
// with that device current and kept in scratch_ptr[]; only that address is
// ever passed to a kernel.
//
// All calls on one GPU share its array.  The backward writes every partial
// row it later reads, so nothing needs clearing between calls, but calls that
// overlap on one GPU (two streams, two threads) race on the array.
#include <mutex>

#include "common.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace {

static __device__ __align__(256) float scratch[TS_RMSNORM_BWD_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};

// The device `stream` belongs to (the current device for the null stream).
int stream_device(hipStream_t stream, int* device) {
  if (stream != nullptr && hipStreamGetDevice(stream, device) == hipSuccess) return TS_OK;
  if (hipGetDevice(device) != hipSuccess) {
    set_error("ts_rmsnorm_bwd_noalloc: no current device");
    return TS_ERR_DEVICE;
  }
  return TS_OK;
}

// The device address of `scratch` on `device`, looked up on the first call for
// that device with the device current.
int scratch_address(int device, void** out) {
  if (device < 0 || device >= kMaxDevices) {
    set_error("ts_rmsnorm_bwd_noalloc: device %d out of range", device);
    return TS_ERR_DEVICE;
  }
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (scratch_ptr[device] == nullptr) {
    int current = -1;
    if (hipGetDevice(&current) != hipSuccess) current = -1;
    if (current != device && hipSetDevice(device) != hipSuccess) {
      set_error("ts_rmsnorm_bwd_noalloc: cannot make device %d current", device);
      return TS_ERR_DEVICE;
    }
    void* ptr = nullptr;
    const hipError_t status = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (current >= 0 && current != device) (void)hipSetDevice(current);
    if (status != hipSuccess || ptr == nullptr) {
      set_error("ts_rmsnorm_bwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", device,
                hipGetErrorString(status));
      return TS_ERR_LAUNCH;
    }
    scratch_ptr[device] = ptr;
  }
  *out = scratch_ptr[device];
  return TS_OK;
}

}  // namespace
}  // namespace ts

extern "C" int ts_rmsnorm_bwd_noalloc(const void* dy, const void* x, const void* w,
                                      const float* rstd, void* dx, void* dw, int64_t rows,
                                      int64_t width, int dtype, void* stream) {
  TS_CHECK_ARG(dy && x && w && rstd, "ts_rmsnorm_bwd_noalloc: null pointer");
  TS_CHECK_ARG(rows >= 0 && width > 0 && width <= (1 << 24),
               "ts_rmsnorm_bwd_noalloc: bad shape rows=%lld width=%lld", (long long)rows,
               (long long)width);
  const int64_t need = dw != nullptr ? ts_rmsnorm_bwd_workspace(rows, width) : 0;
  TS_CHECK_ARG(need <= (int64_t)TS_RMSNORM_BWD_SCRATCH_BYTES,
               "ts_rmsnorm_bwd_noalloc: rows=%lld width=%lld need %lld bytes of dW partials, "
               "more than the %lld-byte scratch array (use ts_rmsnorm_bwd with a workspace)",
               (long long)rows, (long long)width, (long long)need,
               (long long)TS_RMSNORM_BWD_SCRATCH_BYTES);
  void* part = nullptr;
  if (need > 0) {
    int device = 0;
    int status = ts::stream_device((hipStream_t)stream, &device);
    if (status != TS_OK) return status;
    status = ts::scratch_address(device, &part);
    if (status != TS_OK) return status;
  }
  return ts_rmsnorm_bwd(dy, x, w, rstd, dx, dw, part, need, rows, width, dtype, stream);
}
