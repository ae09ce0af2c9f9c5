// Shared device helpers for the gfx950 kernels of libthundersync_hip.
//
// Everything here is written for CDNA4 (gfx950): 64-lane wavefronts, the
// bf16 MFMA instructions v_mfma_f32_16x16x32_bf16 / v_mfma_f32_32x32x16_bf16,
// and 160 KB of LDS per CU.  No other target is built.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>
#include <string.h>
#include <stdio.h>
#include <stdarg.h>

namespace ts {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// dtype codes shared with the host (include/thundersync_hip.h).
enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

// ---------------------------------------------------------------------------
// scalar conversions.  bf16 rounding is round-to-nearest-even (the hardware
// conversion), the rounding torch applies in `.to(torch.bfloat16)`.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf_bits_to_f(uint32_t h) {
  return __uint_as_float(h << 16);
}
__device__ __forceinline__ uint32_t f_to_bf_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // NaN stays NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f(f16 x) { return (float)x; }

template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_f<f16>(float x) { return (f16)x; }

// pack two floats into one dword of two bf16 (lo = a, hi = b), rounded to
// nearest even by gfx950's v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf2(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const bf16x2 h = __builtin_convertvector((f32x2{a, b}), bf16x2);
  uint32_t r;
  __builtin_memcpy(&r, &h, 4);
  return r;
}

// ---------------------------------------------------------------------------
// MFMA wrappers (gfx950).
//
// v_mfma_f32_16x16x32_bf16:  D[16x16] += A[16x32] * B[32x16]
//   A: lane l holds row (l & 15), eight k values of k-group (l >> 4)
//   B: lane l holds col (l & 15), eight k values of k-group (l >> 4)
//   D: lane l holds col (l & 15), rows 4*(l >> 4) + i, i = 0..3
// The contraction pairs A and B through the same (k-group, slot) position,
// so callers may assign any permutation of their contraction index to the
// slots provided A and B use the same one.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_32x32x16_bf16:  D[32x32] += A[32x16] * B[16x32]
//   A: lane l holds row (l & 31), eight k values of k-group (l >> 5)
//   B: lane l holds col (l & 31), eight k values of k-group (l >> 5)
//   D: lane l holds col (l & 31), rows 8*(i >> 2) + 4*(l >> 5) + (i & 3)
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// The same products for a 16-bit element type T (bf16 or f16).  Operands
// travel as bf16x8 bit containers whatever T is (loads, LDS and DMA move bits);
// for f16 they are reinterpreted here, at the instruction that reads them.
template <typename T> __device__ __forceinline__ f32x4 mma16(bf16x8 a, bf16x8 b, f32x4 c) {
  if constexpr (std::is_same_v<T, f16>)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  else
    return mfma16(a, b, c);
}
template <typename T> __device__ __forceinline__ f32x16 mma32(bf16x8 a, bf16x8 b, f32x16 c) {
  if constexpr (std::is_same_v<T, f16>)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  else
    return mfma32(a, b, c);
}

// two floats as one dword of two T values (lo = a, hi = b), rounded to nearest even
template <typename T> __device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (std::is_same_v<T, f16>) {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f16x2 h = __builtin_convertvector((f32x2{a, b}), f16x2);
    uint32_t r;
    __builtin_memcpy(&r, &h, 4);
    return r;
  } else {
    return pack_bf2(a, b);
  }
}

// the float value of 16 bits of T
template <typename T> __device__ __forceinline__ float bits_to_f(uint32_t h) {
  if constexpr (std::is_same_v<T, f16>) return (float)__builtin_bit_cast(f16, (uint16_t)h);
  else return bf_bits_to_f(h);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) {
  bf16x8 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}
__device__ __forceinline__ u32x4 as_u32x4(bf16x8 v) {
  u32x4 r;
  __builtin_memcpy(&r, &v, 16);
  return r;
}

// Transpose an 8x8 block of 16-bit values held as eight 16-byte rows.
// in[j] holds row j (8 columns); out[e] receives column e (8 rows).
__device__ __forceinline__ void transpose8x8(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t x = in[2 * q][p];
      const uint32_t y = in[2 * q + 1][p];
      // column 2p is the low halves, column 2p+1 the high halves
      out[2 * p][q] = __builtin_amdgcn_perm(y, x, 0x05040100u);
      out[2 * p + 1][q] = __builtin_amdgcn_perm(y, x, 0x07060302u);
    }
  }
}

// ---------------------------------------------------------------------------
// buffer resources and direct-to-LDS loads
//
// A raw buffer resource (stride 0) covers `bytes` bytes from `base`; a load
// whose per-lane byte offset is at or past `bytes` is out of range, touches no
// memory and returns zeros (for the LDS form: writes zeros to LDS).  Word 3 is
// gfx9's raw-buffer descriptor: data format 32, no swizzle, no index add.
// ---------------------------------------------------------------------------
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// A read-only table viewed through the constant address space: loads at
// wave-uniform indices become scalar loads (SGPR results), which buffer
// resources and LDS DMA bases require.  Only for memory no kernel writes.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(4))) T* uniform_table(const T* p) {
  return (const __attribute__((address_space(4))) T*)p;
}
// Element i of a read-only table of dword-sized-multiple structs, loaded as
// above (use at wave-uniform indices).
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p, int64_t i) {
  static_assert(sizeof(T) % 4 == 0, "dword-multiple structs only");
  const __attribute__((address_space(4))) uint32_t* q =
      (const __attribute__((address_space(4))) uint32_t*)(p + i);
  uint32_t w[sizeof(T) / 4];
#pragma unroll
  for (int k = 0; k < (int)(sizeof(T) / 4); ++k) w[k] = q[k];
  T v;
  __builtin_memcpy(&v, w, sizeof(T));
  return v;
}
typedef __attribute__((address_space(3))) void lds_void;
constexpr int kRawBufferWord3 = 0x00020000;

// `base` and `bytes` must be wave-uniform; they are read from lane 0 so that
// the descriptor lives in SGPRs even where the compiler cannot prove
// uniformity (no per-lane waterfall loop around the loads).
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  const uint32_t n = __builtin_amdgcn_readfirstlane(bytes);
  return __builtin_amdgcn_make_buffer_rsrc((void*)(((uint64_t)hi << 32) | lo), (short)0, (int)n,
                                           kRawBufferWord3);
}
// 16 bytes per lane from base + voffset into LDS: lane i writes lds + 16 i.
// `lds` must be wave-uniform.
__device__ __forceinline__ void buffer_dma16(rsrc_t r, void* lds, int voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voffset, 0, 0, 0);
}

// buffer_dma16 with the immediate instruction offset OFF, which the hardware
// adds to the LDS address as well as to the global one (pinned by the probe
// test): lane i writes lds + OFF + 16 i from base + voffset + OFF, so DMA
// instructions whose LDS and global offsets advance together share one M0.
template <int OFF>
__device__ __forceinline__ void buffer_dma16_at(rsrc_t r, void* lds, int voffset) {
  static_assert(OFF >= 0 && OFF < 4096, "a 12-bit instruction offset");
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds, 16, voffset, 0, OFF, 0);
}

// A raw buffer descriptor as four SGPR words (base[31:0]; base[47:32] with
// stride 0; num_records; word 3 as above).  `base` and `bytes` must be
// wave-uniform.
__device__ __forceinline__ u32x4 raw_descriptor(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  const uint32_t w0 = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t w1 = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xffffu;
  const uint32_t w2 = (uint32_t)__builtin_amdgcn_readfirstlane(bytes);
  return u32x4{w0, w1, w2, (uint32_t)kRawBufferWord3};
}

// 16 bytes per lane from the descriptor's base + voffset into LDS (lane i
// writes lds + 16 i), issued so that the compiler does not track it: no wait
// is inserted for it anywhere, and the caller accounts for it with explicit
// vmcnt waits (it counts as one vector-memory instruction of the issuing
// wave) and a barrier before other waves read the data.  `lds` must be
// wave-uniform; M0 carries it.
__device__ __forceinline__ void buffer_dma16_untracked(u32x4 desc, void* lds, int voffset) {
  // the LDS address is wave-uniform; readfirstlane keeps it in an SGPR
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voffset), "s"(desc)
               : "memory", "m0");
}

// buffer_dma16_untracked with the non-temporal hint: for a stream read once
__device__ __forceinline__ void buffer_dma16_untracked_nt(u32x4 desc, void* lds, int voffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :
               : "s"(m0), "v"(voffset), "s"(desc)
               : "memory", "m0");
}

// ---------------------------------------------------------------------------
// wave reductions over lanes that differ in the given xor masks
// ---------------------------------------------------------------------------
__device__ __forceinline__ float shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, kWave);
}
// Reductions over the four 16-lane rows of a wave at one position in the row
// (lanes l, l ^ 16, l ^ 32, l ^ 48) with gfx950's lane-swap instructions,
// which are VALU operations (no LDS round trip as with ds_bpermute).
// v_permlane16_swap of a value with itself returns the rows as (0, 0, 2, 2)
// and (1, 1, 3, 3), v_permlane32_swap the halves as (lo, lo) and (hi, hi);
// every lane therefore combines the same operands in the same order.
__device__ __forceinline__ float rows_max4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum4(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// ---------------------------------------------------------------------------
// eight consecutive elements as fp32
// ---------------------------------------------------------------------------
// load / store eight consecutive elements (16 bytes for 16-bit types)
template <typename T> __device__ __forceinline__ void load8(const T* p, float (&o)[8]);
template <> __device__ __forceinline__ void load8<bf16>(const bf16* p, float (&o)[8]) {
  const u32x4 r = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(r[i] << 16);
    o[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void load8<f16>(const f16* p, float (&o)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 r = *reinterpret_cast<const h8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (float)r[i];
}
template <> __device__ __forceinline__ void load8<float>(const float* p, float (&o)[8]) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[i] = a[i];
    o[4 + i] = b[i];
  }
}
template <typename T> __device__ __forceinline__ void store8(T* p, const float (&o)[8]);
template <> __device__ __forceinline__ void store8<bf16>(bf16* p, const float (&o)[8]) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf2(o[2 * i], o[2 * i + 1]);
  *reinterpret_cast<u32x4*>(p) = r;
}
template <> __device__ __forceinline__ void store8<f16>(f16* p, const float (&o)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (f16)o[i];
  *reinterpret_cast<h8*>(p) = r;
}
template <> __device__ __forceinline__ void store8<float>(float* p, const float (&o)[8]) {
  f32x4 a, b;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[i] = o[i];
    b[i] = o[4 + i];
  }
  *reinterpret_cast<f32x4*>(p) = a;
  *reinterpret_cast<f32x4*>(p + 4) = b;
}

// ---------------------------------------------------------------------------
// host-side error state
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int check_launch(const char* what);

// launch kernel<f16> or kernel<bf16> by a DType code (kF16: f16, otherwise bf16)
#define TS_LAUNCH_E(dtype, kernel, ...)                                  \
  do {                                                                   \
    if ((dtype) == ::ts::kF16) hipLaunchKernelGGL((kernel<::ts::f16>), __VA_ARGS__);  \
    else hipLaunchKernelGGL((kernel<::ts::bf16>), __VA_ARGS__);          \
  } while (0)

// the same with further template arguments after the element type
#define TS_LAUNCH_E_T(dtype, kernel, A1, ...)                                                \
  do {                                                                                       \
    if ((dtype) == ::ts::kF16) hipLaunchKernelGGL((kernel<::ts::f16, A1>), __VA_ARGS__);     \
    else hipLaunchKernelGGL((kernel<::ts::bf16, A1>), __VA_ARGS__);                          \
  } while (0)

// out [rows, dim] (bf16) = lhs [rows, vocab] . W [vocab, dim] on the MFMA core
// (the logprob grad-hidden GEMM), launches timed under `label` and, for the
// split-sum pass, `reduce_label`.  Defined in logprob.hip; the C entry
// ts_logprob_grad_hidden documents the arguments.
int grad_hidden_launch(const void* dlogits, int64_t ld_dlogits, const void* weight, int64_t ld_weight, int64_t rows,
                       int64_t dim, int64_t vocab, void* grad_hidden, int64_t ld_grad, void* workspace,
                       int64_t workspace_bytes, int dtype, void* stream, const char* label,
                       const char* reduce_label);

}  // namespace ts

#define TS_CHECK_ARG(cond, ...)            \
  do {                                     \
    if (!(cond)) {                         \
      ::ts::set_error(__VA_ARGS__);        \
      return TS_ERR_INVALID;               \
    }                                      \
  } while (0)
