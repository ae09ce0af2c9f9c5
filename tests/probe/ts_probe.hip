// Test-only hardware probes: one-wave kernels that pin the lane layouts and
// LDS behaviour the library's kernels assume (MFMA operand/result layouts,
// the 8x8 register transpose, LDS DMA, transposed LDS reads, buffer range
// checks, cross-row lane swaps).  Built into tests/probe/libts_probe.so, a
// library of its own: none of this is part of the operator library.
// Every access of every kernel stays inside the 64-lane buffers the
// entry points document.
#include "../../thundersync_amd/csrc/common.h"

namespace ts {

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

// One wave: (1) global_load_lds_dwordx4 with lane i loading src[perm[i]]
// into a 1 KB LDS block, read back in LDS order; (2) ds_read_b64_tr_b16 with
// lane i addressing byte 8 * i of an LDS block holding 16-bit values 0..511;
// (3) buffer_load_dwordx4 ... lds through a buffer resource over the first
// `valid_bytes` of src, lane i at byte offset 16 * perm[i]: lanes whose offset
// is at or past valid_bytes are out of range, read nothing and must leave
// zeros in LDS.  All LDS accesses stay inside their 1 KB blocks and every
// in-range global read lies inside src (64 x 16 bytes).
__global__ __launch_bounds__(64) void probe_lds_kernel(const u32x4* __restrict__ src,
                                                       const int* __restrict__ perm,
                                                       u32x4* __restrict__ dma_out,
                                                       u32x2* __restrict__ tr_out,
                                                       u32x4* __restrict__ buf_out, int valid_bytes) {
  __shared__ __attribute__((aligned(16))) u32x4 block[64];
  __shared__ __attribute__((aligned(16))) u32x4 block2[64];
  __shared__ __attribute__((aligned(16))) uint16_t vals[512];
  const int l = threadIdx.x;
  __builtin_amdgcn_global_load_lds((const void*)(src + perm[l]),
                                   (__attribute__((address_space(3))) void*)block, 16, 0, 0);
  block2[l] = u32x4{0xdeadbeefu, 0xdeadbeefu, 0xdeadbeefu, 0xdeadbeefu};
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  buffer_dma16(make_rsrc(src, (uint32_t)valid_bytes), block2, 16 * perm[l]);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  dma_out[l] = block[l];
  buf_out[l] = block2[l];
  for (int i = l; i < 512; i += 64) vals[i] = (uint16_t)i;
  __syncthreads();
  typedef short i16x4 __attribute__((ext_vector_type(4)));
  i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(vals + 4 * l));
  u32x2 o;
  __builtin_memcpy(&o, &r, 8);
  tr_out[l] = o;
}

// One wave: a buffer_load_dwordx4 ... lds with instruction offset 1024 (the
// builtin's immediate offset), lane i at voffset 16 i, into a 2 KB LDS block
// prefilled with 0xdeadbeef, copied to out (2 KB).  The resource covers all
// of src (128 x 16 bytes); every global byte read lies inside it (1024 +
// 16 i + 16 <= 2048) and every LDS byte written inside the block whether
// the offset moves the LDS address too or not.
__global__ __launch_bounds__(64) void probe_dma_offset_kernel(const u32x4* __restrict__ src,
                                                              u32x4* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) u32x4 block[128];
  const int l = threadIdx.x;
  block[l] = u32x4{0xdeadbeefu, 0xdeadbeefu, 0xdeadbeefu, 0xdeadbeefu};
  block[64 + l] = u32x4{0xdeadbeefu, 0xdeadbeefu, 0xdeadbeefu, 0xdeadbeefu};
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(src, 128 * 16), (lds_void*)block, 16, 16 * l, 0, 1024, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  out[l] = block[l];
  out[64 + l] = block[64 + l];
}

// out[0:64] rows_max4, out[64:128] rows_sum4 of in[lane]; out[128:192] and
// out[192:256] the two results of v_permlane16_swap(in, in), out[256:320]
// and out[320:384] those of v_permlane32_swap(in, in)
__global__ void probe_lanes_kernel(const float* __restrict__ in, float* __restrict__ out) {
  const int l = threadIdx.x;
  const float x = in[l];
  out[l] = rows_max4(x);
  out[64 + l] = rows_sum4(x);
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  out[128 + l] = __uint_as_float(a[0]);
  out[192 + l] = __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  out[256 + l] = __uint_as_float(b[0]);
  out[320 + l] = __uint_as_float(b[1]);
}

}  // namespace ts

namespace {
thread_local char g_probe_error[256] = "";

int launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  snprintf(g_probe_error, sizeof(g_probe_error), "%s: %s", what, hipGetErrorString(e));
  return 2;
}

int refuse(const char* what) {
  snprintf(g_probe_error, sizeof(g_probe_error), "%s", what);
  return 1;
}
}  // namespace

extern "C" {

const char* ts_probe_last_error(void) { return g_probe_error; }

// Entry points (status 0 on success, 1 for a refused argument, 2 for a
// failed launch; ts_probe_last_error() says which):
// Runs one v_mfma_f32_16x16x32_bf16 and one v_mfma_f32_32x32x16_bf16 on
// operands the caller lays out per lane (a, b: 64 lanes x 8 bf16 each), and
// the 8x8 16-bit register transpose on `t_in` (64 lanes x 8 x 8 bf16).
// Writes d16: 64 x 4 fp32, d32: 64 x 16 fp32, t_out: 64 x 8 x 8 bf16.
// Used by the test suite to pin the lane layouts the kernels assume.
// int ts_probe_layouts(const void* a, const void* b, float* d16, float* d32,
//                      const void* t_in, void* t_out, void* stream);
//
// Runs, in one wave, a global_load_lds_dwordx4 in which lane i loads the
// 16 bytes src[perm[i]] (src: 64 x 16 bytes, perm: 64 ints in [0, 64)) and
// copies the resulting 1 KB LDS block to dma_out, then a ds_read_b64_tr_b16
// in which lane i addresses element 4 i of an LDS array holding the 16-bit
// values 0..511, writing each lane's four values to tr_out (64 x 8 bytes),
// then a buffer_load_dwordx4 ... lds through a raw buffer resource over the
// first valid_bytes (0..1024) of src, lane i at byte offset 16 perm[i], into
// an LDS block prefilled with 0xdeadbeef, copied to buf_out (1 KB): lanes
// whose offset is at or past valid_bytes are out of range and must leave
// zeros.  Used by the test suite to pin gfx950's LDS DMA, transpose-read and
// buffer range-check behaviour.
// int ts_probe_lds(const void* src, const int* perm, void* dma_out, void* tr_out, void* buf_out,
//                  int valid_bytes, void* stream);
//
// Runs, in one wave over in[0..63], the cross-row reductions the kernels use
// (maximum and sum over lanes l, l ^ 16, l ^ 32, l ^ 48 by v_permlane16_swap
// and v_permlane32_swap) and the raw swaps.  Writes out[0..383]: the maximum,
// the sum, the two results of v_permlane16_swap(in, in) and the two of
// v_permlane32_swap(in, in), 64 floats each.  Used by the test suite to pin
// the lane semantics.
// int ts_probe_lanes(const float* in, float* out, void* stream);
//
// Runs, in one wave, a buffer_load_dwordx4 ... lds with immediate
// instruction offset 1024, lane i at voffset 16 i, through a raw buffer
// resource over src (128 x 16 bytes) into a 2 KB LDS block prefilled with
// 0xdeadbeef, and copies the block to out (2 KB).  Used by the test suite to
// pin whether the instruction offset moves the LDS address as well as the
// global one.
// int ts_probe_dma_offset(const void* src, void* out, void* stream);

int ts_probe_layouts(const void* a, const void* b, float* d16, float* d32,
                     const void* t_in, void* t_out, void* stream) {
  if (!(a && b && d16 && d32 && t_in && t_out)) return refuse("ts_probe_layouts: null pointer");
  hipLaunchKernelGGL(ts::probe_layouts_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const ts::u32x4*)a, (const ts::u32x4*)b, d16, d32,
                     (const ts::u32x4*)t_in, (ts::u32x4*)t_out);
  return launched("ts_probe_layouts");
}

int ts_probe_lanes(const float* in, float* out, void* stream) {
  if (!(in && out)) return refuse("ts_probe_lanes: null pointer");
  hipLaunchKernelGGL(ts::probe_lanes_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, in, out);
  return launched("ts_probe_lanes");
}

int ts_probe_lds(const void* src, const int* perm, void* dma_out, void* tr_out, void* buf_out,
                 int valid_bytes, void* stream) {
  if (!(src && perm && dma_out && tr_out && buf_out)) return refuse("ts_probe_lds: null pointer");
  if (!(valid_bytes >= 0 && valid_bytes <= 64 * 16)) return refuse("ts_probe_lds: valid_bytes outside [0, 1024]");
  hipLaunchKernelGGL(ts::probe_lds_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const ts::u32x4*)src, perm, (ts::u32x4*)dma_out, (ts::u32x2*)tr_out,
                     (ts::u32x4*)buf_out, valid_bytes);
  return launched("ts_probe_lds");
}

int ts_probe_dma_offset(const void* src, void* out, void* stream) {
  if (!(src && out)) return refuse("ts_probe_dma_offset: null pointer");
  hipLaunchKernelGGL(ts::probe_dma_offset_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                     (const ts::u32x4*)src, (ts::u32x4*)out);
  return launched("ts_probe_dma_offset");
}

}  // extern "C"
