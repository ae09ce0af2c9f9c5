// Boundary-adjoint reduction and FP32 ledger accumulation for gfx950.
//
// Reference: engine/boundary_adjoint.py:49-115 -- the fused reduction of up to
// 16 consumer adjoints into an optional existing parent adjoint, accumulated
// in fp32 in input order (existing first, then the adjoints) and cast once to
// the input dtype -- and engine/streaming.py:2647-2665 -- the FP32 ledger: the
// first contribution is widened into it, later ones are added after exact
// widening (a mixed-dtype add_).
//
// Bandwidth-bound: every input element is read once and every output element
// written once, eight elements per thread with 16-byte accesses; the number of
// adjoints is a template parameter, so a thread issues all of its loads before
// the first add (a runtime-bounded loop would wait for each load in turn).  A
// size that is not a multiple of eight leaves a scalar tail to the last thread.
// Inputs are read with non-temporal loads (each byte is used once) by
// 128-thread blocks: on the 16-adjoint bf16 reduction that pair runs about 12%
// faster than cached loads in 256-thread blocks.
#include <type_traits>

#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace {

constexpr int kThreads = 128;
constexpr int kMaxAdjoints = 16;

struct AdjointPtrs {
  const void* p[kMaxAdjoints];
};

// eight elements from 16-byte aligned p (32 bytes for float), non-temporal
template <typename T> __device__ __forceinline__ void load8_once(const T* p, float (&o)[8]) {
  const u32x4* q = reinterpret_cast<const u32x4*>(p);
  const u32x4 r = __builtin_nontemporal_load(q);
  if constexpr (sizeof(T) == 4) {
    const u32x4 r2 = __builtin_nontemporal_load(q + 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] = __uint_as_float(r[i]);
      o[4 + i] = __uint_as_float(r2[i]);
    }
  } else if constexpr (std::is_same<T, bf16>::value) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(r[i] << 16);
      o[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  } else {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const h8 h = __builtin_bit_cast(h8, r);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (float)h[i];
  }
}

template <typename T> __device__ __forceinline__ float load1(const T* p);
template <> __device__ __forceinline__ float load1<bf16>(const bf16* p) {
  return __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
}
template <> __device__ __forceinline__ float load1<f16>(const f16* p) { return (float)*p; }
template <> __device__ __forceinline__ float load1<float>(const float* p) { return *p; }

template <typename T> __device__ __forceinline__ void store1(T* p, float v);
template <> __device__ __forceinline__ void store1<bf16>(bf16* p, float v) { *p = (bf16)v; }
template <> __device__ __forceinline__ void store1<f16>(f16* p, float v) { *p = (f16)v; }
template <> __device__ __forceinline__ void store1<float>(float* p, float v) { *p = v; }

// out[i] = cast(existing[i] + a_0[i] + ... + a_{N-1}[i]), the sum in fp32 and
// in that order (existing absent: 0 + a_0 + ...)
template <typename T, int N, bool EXISTING>
__global__ __launch_bounds__(kThreads) void adjoint_reduce_kernel(AdjointPtrs a, const T* __restrict__ existing,
                                                                  T* __restrict__ out, int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 8;
  if (i0 + 8 <= n) {
    float v[N + 1][8];
    if (EXISTING) load8_once(existing + i0, v[N]);
#pragma unroll
    for (int k = 0; k < N; ++k) load8_once(static_cast<const T*>(a.p[k]) + i0, v[k]);
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = EXISTING ? v[N][e] : 0.f;
#pragma unroll
    for (int k = 0; k < N; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] += v[k][e];
    store8(out + i0, acc);
  } else if (i0 < n) {
    for (int64_t i = i0; i < n; ++i) {
      float acc = EXISTING ? load1(existing + i) : 0.f;
#pragma unroll
      for (int k = 0; k < N; ++k) acc += load1(static_cast<const T*>(a.p[k]) + i);
      store1(out + i, acc);
    }
  }
}

// INIT: ledger = widen(c); else ledger += widen(c)
template <typename T, bool INIT>
__global__ __launch_bounds__(kThreads) void ledger_add_kernel(float* __restrict__ ledger,
                                                              const T* __restrict__ c, int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 8;
  if (i0 + 8 <= n) {
    float x[8], l[8];
    load8_once(c + i0, x);
    if (!INIT) load8(ledger + i0, l);
#pragma unroll
    for (int e = 0; e < 8; ++e) l[e] = INIT ? x[e] : l[e] + x[e];
    store8(ledger + i0, l);
  } else if (i0 < n) {
    for (int64_t i = i0; i < n; ++i) ledger[i] = INIT ? load1(c + i) : ledger[i] + load1(c + i);
  }
}

dim3 grid_of(int64_t n) { return dim3((unsigned)((n + 8 * kThreads - 1) / (8 * kThreads))); }

template <typename T, int N>
void launch_reduce(const AdjointPtrs& a, const void* existing, void* out, int64_t n, hipStream_t s) {
  TimedLaunch timed_("adjoint.reduce_kernel", s);
  if (existing)
    hipLaunchKernelGGL((adjoint_reduce_kernel<T, N, true>), grid_of(n), dim3(kThreads), 0, s, a,
                       static_cast<const T*>(existing), static_cast<T*>(out), n);
  else
    hipLaunchKernelGGL((adjoint_reduce_kernel<T, N, false>), grid_of(n), dim3(kThreads), 0, s, a,
                       static_cast<const T*>(existing), static_cast<T*>(out), n);
}

template <typename T, int N = 0>
void dispatch_reduce(int count, const AdjointPtrs& a, const void* existing, void* out, int64_t n, hipStream_t s) {
  if constexpr (N <= kMaxAdjoints) {
    if (count == N) return launch_reduce<T, N>(a, existing, out, n, s);
    dispatch_reduce<T, N + 1>(count, a, existing, out, n, s);
  }
}

bool ok16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace ts

extern "C" {

int ts_adjoint_reduce(const void* const* adjoints, int n_adjoints, const void* existing, void* out,
                      int64_t n_elements, int dtype, void* stream) {
  using namespace ts;
  TS_CHECK_ARG(n_adjoints >= 0 && n_adjoints <= kMaxAdjoints && (n_adjoints > 0 || existing),
               "ts_adjoint_reduce: %d adjoints (0..%d, and an existing adjoint when 0)", n_adjoints,
               kMaxAdjoints);
  TS_CHECK_ARG(dtype == TS_F32 || dtype == TS_F16 || dtype == TS_BF16, "ts_adjoint_reduce: dtype %d", dtype);
  TS_CHECK_ARG(n_elements >= 0, "ts_adjoint_reduce: n_elements %lld", (long long)n_elements);
  if (n_elements == 0) return TS_OK;  // nothing is read or written: pointers may be null
  TS_CHECK_ARG(out && ok16(out) && (!existing || ok16(existing)),
               "ts_adjoint_reduce: out/existing must be 16-byte aligned (n_elements=%lld)",
               (long long)n_elements);
  TS_CHECK_ARG(n_adjoints == 0 || adjoints, "ts_adjoint_reduce: null adjoint table");
  AdjointPtrs a{};
  for (int k = 0; k < n_adjoints; ++k) {
    TS_CHECK_ARG(adjoints[k] && ok16(adjoints[k]), "ts_adjoint_reduce: adjoint %d null or not 16-byte aligned", k);
    TS_CHECK_ARG(adjoints[k] != out && existing != out, "ts_adjoint_reduce: out aliases an input");
    a.p[k] = adjoints[k];
  }
  TS_CHECK_ARG(existing != out, "ts_adjoint_reduce: out aliases an input");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == TS_F32) dispatch_reduce<float>(n_adjoints, a, existing, out, n_elements, s);
  else if (dtype == TS_F16) dispatch_reduce<f16>(n_adjoints, a, existing, out, n_elements, s);
  else dispatch_reduce<bf16>(n_adjoints, a, existing, out, n_elements, s);
  return check_launch("ts_adjoint_reduce");
}

int ts_ledger_add(float* ledger, const void* contribution, int64_t n_elements, int dtype, int init, void* stream) {
  using namespace ts;
  TS_CHECK_ARG(dtype == TS_F32 || dtype == TS_F16 || dtype == TS_BF16, "ts_ledger_add: dtype %d", dtype);
  TS_CHECK_ARG(n_elements >= 0, "ts_ledger_add: n_elements %lld", (long long)n_elements);
  if (n_elements == 0) return TS_OK;  // nothing is read or written: pointers may be null
  TS_CHECK_ARG(ledger && contribution && ok16(ledger) && ok16(contribution) && (const void*)ledger != contribution,
               "ts_ledger_add: ledger/contribution null, aliased or not 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  TimedLaunch timed_("adjoint.ledger_kernel", s);
  const dim3 g = grid_of(n_elements);
  if (dtype == TS_F32) {
    if (init) hipLaunchKernelGGL((ledger_add_kernel<float, true>), g, dim3(kThreads), 0, s, ledger, (const float*)contribution, n_elements);
    else hipLaunchKernelGGL((ledger_add_kernel<float, false>), g, dim3(kThreads), 0, s, ledger, (const float*)contribution, n_elements);
  } else if (dtype == TS_F16) {
    if (init) hipLaunchKernelGGL((ledger_add_kernel<f16, true>), g, dim3(kThreads), 0, s, ledger, (const f16*)contribution, n_elements);
    else hipLaunchKernelGGL((ledger_add_kernel<f16, false>), g, dim3(kThreads), 0, s, ledger, (const f16*)contribution, n_elements);
  } else {
    if (init) hipLaunchKernelGGL((ledger_add_kernel<bf16, true>), g, dim3(kThreads), 0, s, ledger, (const bf16*)contribution, n_elements);
    else hipLaunchKernelGGL((ledger_add_kernel<bf16, false>), g, dim3(kThreads), 0, s, ledger, (const bf16*)contribution, n_elements);
  }
  return check_launch("ts_ledger_add");
}

}  // extern "C"
