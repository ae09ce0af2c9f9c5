// Library identity, error reporting and the lane-layout probe.
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

// One wave: a 16x16x32 and a 32x32x16 MFMA on caller-laid-out operands, and
// the register transpose used to feed transposed operands from LDS rows.
__global__ __launch_bounds__(64) void probe_layouts_kernel(
    const u32x4* __restrict__ a, const u32x4* __restrict__ b, float* __restrict__ d16,
    float* __restrict__ d32, const u32x4* __restrict__ t_in, u32x4* __restrict__ t_out) {
  const int l = threadIdx.x;
  const bf16x8 av = as_bf16x8(a[l]);
  const bf16x8 bv = as_bf16x8(b[l]);
  f32x4 c4 = {0.f, 0.f, 0.f, 0.f};
  c4 = mfma16(av, bv, c4);
  for (int i = 0; i < 4; ++i) d16[l * 4 + i] = c4[i];
  f32x16 c16;
  for (int i = 0; i < 16; ++i) c16[i] = 0.f;
  c16 = mfma32(av, bv, c16);
  for (int i = 0; i < 16; ++i) d32[l * 16 + i] = c16[i];
  u32x4 in[8], out[8];
  for (int j = 0; j < 8; ++j) in[j] = t_in[l * 8 + j];
  transpose8x8(in, out);
  for (int j = 0; j < 8; ++j) t_out[l * 8 + j] = out[j];
}

}  // namespace ts

extern "C" {

const char* ts_hip_version(void) { return "thundersync_hip 0.1.0 gfx950"; }

const char* ts_hip_last_error(void) { return ts::g_error; }

int ts_probe_layouts(const void* a, const void* b, float* d16, float* d32,
                     const void* t_in, void* t_out, void* stream) {
  TS_CHECK_ARG(a && b && d16 && d32 && t_in && t_out, "ts_probe_layouts: null pointer");
  hipLaunchKernelGGL(ts::probe_layouts_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const ts::u32x4*)a, (const ts::u32x4*)b, d16, d32,
                     (const ts::u32x4*)t_in, (ts::u32x4*)t_out);
  return ts::check_launch("ts_probe_layouts");
}

}  // extern "C"
