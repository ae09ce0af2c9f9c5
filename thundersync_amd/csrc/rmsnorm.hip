// RMSNorm forward / backward for gfx950.
//
// Bandwidth-bound: every element is read once (forward: x; backward: x, dy)
// and written once, with 16-byte vector accesses.  A row is owned by LPR
// lanes (LPR = 64 for wide rows such as the 4096-wide residual norm, fewer
// for the 128-wide per-head q/k norms so that one wave covers several rows).
// Each lane keeps its NV eight-element vectors of the row in registers, so a
// row is read from HBM once.
//
// Reference semantics: accel/rms_norm.py:9-43 (forward casts, FP32 VJP) and
// grpo/rms_norm_native.py:8-74 (dW = sum over rows of dy * x * rstd in fp32).
#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace {

constexpr int kThreads = 256;  // 4 waves

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

// round a float through T and back
template <typename T> __device__ __forceinline__ float round_t(float x) {
  return to_f(from_f<T>(x));
}

template <int LPR> __device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int m = LPR / 2; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}

// ---------------------------------------------------------------------------
// forward, vector path (width % 8 == 0)
// ---------------------------------------------------------------------------
template <typename T, int LPR, int NV>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_vec(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
    float* __restrict__ rstd, int64_t rows, int width, float eps) {
  constexpr int kRowsPerWave = kWave / LPR;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t row = ((int64_t)blockIdx.x * (kThreads / kWave) + wave) * kRowsPerWave + lane / LPR;
  const int sub = lane % LPR;
  if (row >= rows) return;
  const int nvec = width / 8;
  const T* xr = x + row * width;
  float v[NV][8];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int vi = sub + k * LPR;
    if (vi < nvec) {
      load8<T>(xr + vi * 8, v[k]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = fmaf(v[k][i], v[k][i], ss);
    }
  }
  ss = row_sum<LPR>(ss);
  const float r = __frsqrt_rn(ss / (float)width + eps);
  if (sub == 0) rstd[row] = r;
  T* yr = y + row * width;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int vi = sub + k * LPR;
    if (vi < nvec) {
      float wv[8], o[8];
      load8<T>(w + vi * 8, wv);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = wv[i] * round_t<T>(v[k][i] * r);
      store8<T>(yr + vi * 8, o);
    }
  }
}

// forward, scalar path (any width): one wave per row
template <typename T>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_scalar(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
    float* __restrict__ rstd, int64_t rows, int width, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = (int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave;
  if (row >= rows) return;
  const T* xr = x + row * width;
  float ss = 0.f;
  for (int i = lane; i < width; i += kWave) {
    const float a = to_f(xr[i]);
    ss = fmaf(a, a, ss);
  }
  ss = wave_sum(ss);
  const float r = __frsqrt_rn(ss / (float)width + eps);
  if (lane == 0) rstd[row] = r;
  T* yr = y + row * width;
  for (int i = lane; i < width; i += kWave)
    yr[i] = from_f<T>(to_f(w[i]) * round_t<T>(to_f(xr[i]) * r));
}

// ---------------------------------------------------------------------------
// backward, vector path.  Block b owns rows [b*slab, (b+1)*slab) and writes
// one fp32 partial dW row into part[b]; rmsnorm_dw_reduce sums the partials
// in block order.
// ---------------------------------------------------------------------------
template <typename T, int LPR, int NV>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_vec(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ rstd, T* __restrict__ dx, float* __restrict__ part,
    int64_t rows, int width, int64_t slab, int want_dx, int want_dw) {
  constexpr int kRowsPerWave = kWave / LPR;
  constexpr int kRowsPerPass = (kThreads / kWave) * kRowsPerWave;
  extern __shared__ float lds_dw[];  // [width] when want_dw
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int sub = lane % LPR;
  const int rsub = wave * kRowsPerWave + lane / LPR;  // 0 .. kRowsPerPass-1
  const int nvec = width / 8;
  const int64_t r0 = (int64_t)blockIdx.x * slab;
  const int64_t r1 = min(rows, r0 + slab);

  float wv[NV][8];
  float acc[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int vi = sub + k * LPR;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[k][i] = 0.f;
    if (vi < nvec) load8<T>(w + vi * 8, wv[k]);
  }
  const float inv_w = 1.f / (float)width;
  for (int64_t row = r0 + rsub; row < r1; row += kRowsPerPass) {
    const float r = rstd[row];
    float xv[NV][8], gv[NV][8];
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int vi = sub + k * LPR;
      if (vi < nvec) {
        float dv[8];
        load8<T>(x + row * width + vi * 8, xv[k]);
        load8<T>(dy + row * width + vi * 8, dv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc[k][i] = fmaf(dv[i] * xv[k][i], r, acc[k][i]);
          gv[k][i] = dv[i] * wv[k][i];
          xv[k][i] *= r;  // xhat
          dot = fmaf(gv[k][i], xv[k][i], dot);
        }
      }
    }
    if (want_dx) {
      dot = row_sum<LPR>(dot) * inv_w;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int vi = sub + k * LPR;
        if (vi < nvec) {
          float o[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = r * (gv[k][i] - xv[k][i] * dot);
          store8<T>(dx + row * width + vi * 8, o);
        }
      }
    }
  }
  if (!want_dw) return;
  // fixed-order combine of the block's row groups: group 0 stores, then each
  // later group adds in turn
  for (int g = 0; g < kRowsPerPass; ++g) {
    if (rsub == g) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int vi = sub + k * LPR;
        if (vi < nvec) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float* p = &lds_dw[vi * 8 + i];
            *p = (g == 0) ? acc[k][i] : (*p + acc[k][i]);
          }
        }
      }
    }
    __syncthreads();
  }
  for (int c = threadIdx.x; c < width; c += kThreads) part[(int64_t)blockIdx.x * width + c] = lds_dw[c];
}

// backward, scalar path (any width): the block's 256 threads work on one
// row at a time; thread t owns columns t, t + 256, ... of the dW partial, so
// one LDS row of `width` floats holds it without conflicts between threads.
template <typename T>
__global__ __launch_bounds__(kThreads) void rmsnorm_bwd_scalar(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ rstd, T* __restrict__ dx, float* __restrict__ part,
    int64_t rows, int width, int64_t slab, int want_dx, int want_dw) {
  extern __shared__ float lds_dw[];  // [width] (+ 4 floats for the row sum)
  float* red = lds_dw + width;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t r0 = (int64_t)blockIdx.x * slab;
  const int64_t r1 = min(rows, r0 + slab);
  for (int c = threadIdx.x; c < width; c += kThreads) lds_dw[c] = 0.f;
  const float inv_w = 1.f / (float)width;
  for (int64_t row = r0; row < r1; ++row) {
    const float r = rstd[row];
    const T* xr = x + row * width;
    const T* dr = dy + row * width;
    float dot = 0.f;
    for (int c = threadIdx.x; c < width; c += kThreads) {
      const float d = to_f(dr[c]);
      const float xv = to_f(xr[c]);
      lds_dw[c] = fmaf(d * xv, r, lds_dw[c]);
      dot = fmaf(d * to_f(w[c]), xv * r, dot);
    }
    if (want_dx) {
      dot = wave_sum(dot);
      if (lane == 0) red[wave] = dot;
      __syncthreads();
      dot = (red[0] + red[1] + red[2] + red[3]) * inv_w;
      __syncthreads();
      for (int c = threadIdx.x; c < width; c += kThreads) {
        const float xh = to_f(xr[c]) * r;
        dx[row * width + c] = from_f<T>(r * (to_f(dr[c]) * to_f(w[c]) - xh * dot));
      }
    }
  }
  if (!want_dw) return;
  for (int c = threadIdx.x; c < width; c += kThreads) part[(int64_t)blockIdx.x * width + c] = lds_dw[c];
}

// dW = T(sum over partial rows, in order)
template <typename T>
__global__ __launch_bounds__(kThreads) void rmsnorm_dw_reduce(
    const float* __restrict__ part, T* __restrict__ dw, int nparts, int width) {
  const int c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= width) return;
  float s = 0.f;
  for (int p = 0; p < nparts; ++p) s += part[(int64_t)p * width + c];
  dw[c] = from_f<T>(s);
}

// --------------------------------------------------------------------------
// host dispatch
// --------------------------------------------------------------------------
struct Geometry {
  int lpr;  // lanes per row (vector path); 0 = scalar path
  int nv;   // vectors per lane (1, 2, 4, 8 or 16)
};

Geometry pick(int64_t width, int dtype) {
  Geometry g{0, 0};
  if (width % 8 != 0) return g;
  const int64_t nvec = width / 8;
  int lpr = 64;
  while (lpr > 4 && lpr > nvec) lpr >>= 1;
  const int64_t nv = (nvec + lpr - 1) / lpr;
  int nvp = 1;
  while (nvp < nv) nvp <<= 1;
  if (nvp > 16) return g;  // wider than 8192: scalar path
  (void)dtype;
  g.lpr = lpr;
  g.nv = nvp;
  return g;
}

constexpr int64_t kMaxParts = 256;

int64_t bwd_parts(int64_t rows) {
  // at least 32 rows per block so the partial rows stay a small fraction of
  // the traffic; at most kMaxParts blocks
  int64_t parts = (rows + 31) / 32;
  if (parts > kMaxParts) parts = kMaxParts;
  if (parts < 1) parts = 1;
  return parts;
}

template <typename T>
int launch_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows, int width,
               float eps, hipStream_t s) {
  const Geometry g = pick(width, 0);
  if (g.lpr == 0) {
    const int64_t blocks = (rows + 3) / 4;
    { ts::TimedLaunch timed_("rmsnorm.rmsnorm_fwd_scalar", s); hipLaunchKernelGGL(rmsnorm_fwd_scalar<T>, dim3((unsigned)blocks), dim3(kThreads), 0, s,
                       (const T*)x, (const T*)w, (T*)y, rstd, rows, width, eps); }
    return check_launch("ts_rmsnorm_fwd");
  }
  const int64_t rows_per_block = 4 * (64 / g.lpr);
  const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
#define TS_FWD(LPR, NV)                                                                     \
  if (g.lpr == LPR && g.nv == NV) {                                                         \
    { ts::TimedLaunch timed_("rmsnorm.rmsnorm_fwd_vec", s); hipLaunchKernelGGL((rmsnorm_fwd_vec<T, LPR, NV>), grid, dim3(kThreads), 0, s,           \
                       (const T*)x, (const T*)w, (T*)y, rstd, rows, width, eps); }            \
    return check_launch("ts_rmsnorm_fwd");                                                  \
  }
  TS_FWD(4, 1) TS_FWD(8, 1) TS_FWD(16, 1) TS_FWD(32, 1) TS_FWD(64, 1)
  TS_FWD(4, 2) TS_FWD(8, 2) TS_FWD(16, 2) TS_FWD(32, 2) TS_FWD(64, 2) TS_FWD(64, 4) TS_FWD(64, 8) TS_FWD(64, 16)
#undef TS_FWD
  set_error("ts_rmsnorm_fwd: no kernel for width %d", width);
  return TS_ERR_INVALID;
}

template <typename T>
int launch_bwd(const void* dy, const void* x, const void* w, const float* rstd, void* dx,
               void* dw, float* part, int64_t rows, int width, hipStream_t s) {
  const Geometry g = pick(width, 0);
  const int64_t parts = bwd_parts(rows);
  const int64_t slab = (rows + parts - 1) / parts;
  const int want_dx = dx != nullptr, want_dw = dw != nullptr;
  if (g.lpr == 0) {
    const size_t lds = (size_t)(width + 4) * sizeof(float);
    if (lds > 160 * 1024) {
      set_error("ts_rmsnorm_bwd: width %d too wide for the scalar dW path", width);
      return TS_ERR_INVALID;
    }
    { ts::TimedLaunch timed_("rmsnorm.rmsnorm_bwd_scalar", s); hipLaunchKernelGGL(rmsnorm_bwd_scalar<T>, dim3((unsigned)parts), dim3(kThreads), lds, s,
                       (const T*)dy, (const T*)x, (const T*)w, rstd, (T*)dx, part, rows, width,
                       slab, want_dx, want_dw); }
  } else {
    const size_t lds = want_dw ? (size_t)width * sizeof(float) : 0;
    const dim3 grid((unsigned)parts);
    bool launched = false;
#define TS_BWD(LPR, NV)                                                                      \
  if (!launched && g.lpr == LPR && g.nv == NV) {                                             \
    { ts::TimedLaunch timed_("rmsnorm.rmsnorm_bwd_vec", s); hipLaunchKernelGGL((rmsnorm_bwd_vec<T, LPR, NV>), grid, dim3(kThreads), lds, s,          \
                       (const T*)dy, (const T*)x, (const T*)w, rstd, (T*)dx, part, rows,     \
                       width, slab, want_dx, want_dw); }                                        \
    launched = true;                                                                         \
  }
    TS_BWD(4, 1) TS_BWD(8, 1) TS_BWD(16, 1) TS_BWD(32, 1) TS_BWD(64, 1)
    TS_BWD(4, 2) TS_BWD(8, 2) TS_BWD(16, 2) TS_BWD(32, 2) TS_BWD(64, 2) TS_BWD(64, 4) TS_BWD(64, 8) TS_BWD(64, 16)
#undef TS_BWD
    if (!launched) {
      set_error("ts_rmsnorm_bwd: no kernel for width %d", width);
      return TS_ERR_INVALID;
    }
  }
  int st = check_launch("ts_rmsnorm_bwd");
  if (st != TS_OK || !want_dw) return st;
  { ts::TimedLaunch timed_("rmsnorm.rmsnorm_dw_reduce", s); hipLaunchKernelGGL(rmsnorm_dw_reduce<T>, dim3((unsigned)((width + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, s, (const float*)part, (T*)dw, (int)parts, width); }
  return check_launch("ts_rmsnorm_bwd (dW reduce)");
}

}  // namespace
}  // namespace ts

extern "C" {

int ts_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows,
                   int64_t width, float eps, int dtype, void* stream) {
  TS_CHECK_ARG(x && w && y && rstd, "ts_rmsnorm_fwd: null pointer");
  TS_CHECK_ARG(rows >= 0 && width > 0 && width <= (1 << 24),
               "ts_rmsnorm_fwd: bad shape rows=%lld width=%lld", (long long)rows,
               (long long)width);
  if (rows == 0) return TS_OK;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case TS_BF16: return ts::launch_fwd<ts::bf16>(x, w, y, rstd, rows, (int)width, eps, s);
    case TS_F16: return ts::launch_fwd<ts::f16>(x, w, y, rstd, rows, (int)width, eps, s);
    case TS_F32: return ts::launch_fwd<float>(x, w, y, rstd, rows, (int)width, eps, s);
  }
  ts::set_error("ts_rmsnorm_fwd: unsupported dtype code %d", dtype);
  return TS_ERR_INVALID;
}

int64_t ts_rmsnorm_bwd_workspace(int64_t rows, int64_t width) {
  if (rows <= 0 || width <= 0) return 0;
  return ts::bwd_parts(rows) * width * (int64_t)sizeof(float);
}

int ts_rmsnorm_bwd(const void* dy, const void* x, const void* w, const float* rstd, void* dx,
                   void* dw, void* workspace, int64_t workspace_bytes, int64_t rows,
                   int64_t width, int dtype, void* stream) {
  TS_CHECK_ARG(dy && x && w && rstd, "ts_rmsnorm_bwd: null pointer");
  TS_CHECK_ARG(rows >= 0 && width > 0 && width <= (1 << 24),
               "ts_rmsnorm_bwd: bad shape rows=%lld width=%lld", (long long)rows,
               (long long)width);
  hipStream_t s = (hipStream_t)stream;
  if (rows == 0) {
    if (dw) {
      const int64_t esz = dtype == TS_F32 ? 4 : 2;
      if (hipMemsetAsync(dw, 0, (size_t)(width * esz), s) != hipSuccess)
        return ts::check_launch("ts_rmsnorm_bwd (zero dW)");
    }
    return TS_OK;
  }
  if (dw) {
    const int64_t need = ts_rmsnorm_bwd_workspace(rows, width);
    TS_CHECK_ARG(workspace && workspace_bytes >= need,
                 "ts_rmsnorm_bwd: workspace of %lld bytes, need %lld",
                 (long long)workspace_bytes, (long long)need);
  }
  float* part = (float*)workspace;
  switch (dtype) {
    case TS_BF16:
      return ts::launch_bwd<ts::bf16>(dy, x, w, rstd, dx, dw, part, rows, (int)width, s);
    case TS_F16:
      return ts::launch_bwd<ts::f16>(dy, x, w, rstd, dx, dw, part, rows, (int)width, s);
    case TS_F32:
      return ts::launch_bwd<float>(dy, x, w, rstd, dx, dw, part, rows, (int)width, s);
  }
  ts::set_error("ts_rmsnorm_bwd: unsupported dtype code %d", dtype);
  return TS_ERR_INVALID;
}

}  // extern "C"
