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

// eight consecutive elements kept as loaded (16-bit types: four dwords), so a
// row held across a loop iteration costs half the registers of its floats
template <typename T> struct Packed8 { u32x4 v; };
template <> struct Packed8<float> { f32x4 a, b; };

template <typename T> __device__ __forceinline__ Packed8<T> load_packed(const T* p) {
  return Packed8<T>{*reinterpret_cast<const u32x4*>(p)};
}
template <> __device__ __forceinline__ Packed8<float> load_packed<float>(const float* p) {
  return Packed8<float>{*reinterpret_cast<const f32x4*>(p), *reinterpret_cast<const f32x4*>(p + 4)};
}
// non-temporal: for rows the kernel reads once (the backward's x and dy rows:
// 0.088 -> 0.077 ms on [16384, 4096] bf16 against cached loads)
template <typename T> __device__ __forceinline__ Packed8<T> load_packed_once(const T* p) {
  return Packed8<T>{__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p))};
}
template <> __device__ __forceinline__ Packed8<float> load_packed_once<float>(const float* p) {
  return Packed8<float>{__builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p)),
                        __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + 1)};
}
template <typename T> __device__ __forceinline__ void store_packed(T* p, const Packed8<T>& r) {
  *reinterpret_cast<u32x4*>(p) = r.v;
}
template <> __device__ __forceinline__ void store_packed<float>(float* p, const Packed8<float>& r) {
  *reinterpret_cast<f32x4*>(p) = r.a;
  *reinterpret_cast<f32x4*>(p + 4) = r.b;
}
// hide a value's origin from the optimiser (an empty asm that "changes" it), so
// products formed from it once are formed again rather than kept live
template <typename T> __device__ __forceinline__ Packed8<T> opaque(Packed8<T> r) {
  asm volatile("" : "+v"(r.v));
  return r;
}
template <> __device__ __forceinline__ Packed8<float> opaque<float>(Packed8<float> r) {
  asm volatile("" : "+v"(r.a), "+v"(r.b));
  return r;
}
template <typename T> __device__ __forceinline__ void unpack(const Packed8<T>& r, float (&o)[8]);
template <> __device__ __forceinline__ void unpack<bf16>(const Packed8<bf16>& r, float (&o)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = __uint_as_float(r.v[i] << 16);
    o[2 * i + 1] = __uint_as_float(r.v[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack<f16>(const Packed8<f16>& r, float (&o)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 h = __builtin_bit_cast(h8, r.v);
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = (float)h[i];
}
template <> __device__ __forceinline__ void unpack<float>(const Packed8<float>& r, float (&o)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[i] = r.a[i];
    o[4 + i] = r.b[i];
  }
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
// forward
//
// The primal is byte-identical to transformers' Qwen3RMSNorm on this device:
//   x = float(h); var = x.pow(2).mean(-1); rstd = rsqrt(var + eps);
//   y = w * T(x * rstd)
// (accel/rms_norm.py:11-14 restates the same operations).  Two facts make
// that possible:
//  * torch sums x.pow(2) along a contiguous row in a fixed order that depends
//    only on (rows, width) and the CU count: the schedule of its reduction
//    kernel (ATen/native/hip/Reduce.cuh of the torch 2.10 ROCm build:
//    setReduceConfig, input_vectorized_thread_reduce_impl / thread_reduce_impl,
//    block_x_reduce, block_y_reduce; MeanOps::project = sum * factor).
//    RowReduce below is that schedule; the kernels perform the same fp32
//    additions on the same operands in the same order (no contraction into
//    FMAs anywhere on the variance path);
//  * torch.rsqrt of an fp32 tensor returns the correctly rounded 1/sqrt(x) for
//    every positive finite float -- equal to float(1.0 / sqrt(double(x))),
//    checked bit for bit over all 2^31 - 2^23 of them on an MI355X -- so rstd
//    is computed that way.
// ---------------------------------------------------------------------------

// How torch reduces one row of a contiguous [rows, width] fp32 tensor.
// Thread (x, y) of the row's bw x bh threads sums the loads
//   idx = x + y * ym, idx + step, idx + 2 step, ...
// into four accumulators (load element i -> accumulator i for 4-element
// vector loads; load j -> accumulator j mod 4 for scalar loads), adds them as
// ((a0 + a1) + a2) + a3, then the threads combine: across x first (pairwise
// halving from bw/2 down to 64 in LDS, then v += shfl_down(v, 1, 2, 4, ...)),
// then across y (halving from bh/2 down to 1).
struct RowReduce {
  int vec;   // 1: 4-element vector loads (width >= 128); 0: scalar loads
  int bw;    // threads along the row (power of two, <= 512)
  int bh;    // thread rows splitting the row's inputs (1: not split)
  int ym;    // first load of thread row y is x + y * ym
  int step;  // stride between one thread's loads, in loads
};

// setReduceConfig (Reduce.cuh) for a reduction over the contiguous last dim
// of a [rows, width] fp32 tensor; false where torch would split the row over
// several work-groups (one row wider than 130560), which is not reproduced.
inline bool torch_row_reduce(int64_t rows, int64_t width, int num_cu, RowReduce& c) {
  constexpr int64_t kMaxThreads = 512, kWarp = 64;
  auto last_pow2 = [](int64_t n) {
    int64_t p = 1;
    while (p * 2 <= n) p *= 2;
    return p;
  };
  c.vec = width >= 128;
  const int64_t dim0 = c.vec ? width / 4 : width;
  const int64_t d0 = dim0 < kMaxThreads ? last_pow2(dim0) : kMaxThreads;
  const int64_t d1 = rows < kMaxThreads ? last_pow2(rows) : kMaxThreads;
  int64_t bw = std::min(d0, kWarp);
  const int64_t block_h = std::min(d1, kMaxThreads / bw);
  bw = std::min(d0, kMaxThreads / block_h);
  int64_t step = bw;
  int64_t per_thread = (width + step - 1) / step;
  bool split = per_thread >= std::min<int64_t>(block_h * 16, 256);
  if (rows > 1 && per_thread < 1024 && num_cu < 100) split = false;  // ROCm: force_splitting_output
  c.bh = 1;
  c.ym = 0;
  if (split) {
    c.ym = (int)step;
    step *= block_h;
    c.bh = (int)block_h;
    per_thread = (width + step - 1) / step;
    // a single output row whose threads would still sum >= 256 values each is
    // split across work-groups (global_reduce)
    if (rows == 1 && per_thread >= 256) return false;
  }
  c.bw = (int)bw;
  c.step = (int)step;
  return true;
}

// squares of elements as torch's x.pow(2) of the fp32 copy
__device__ __forceinline__ float sq_rn(float a) {
#pragma clang fp contract(off)
  return a * a;
}
__device__ __forceinline__ float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}
// rstd = rsqrt(var + eps) as torch computes it: var = sum * factor, one fp32
// add of eps, then the correctly rounded reciprocal square root
__device__ __forceinline__ float torch_rstd(float sum, float factor, float eps) {
#pragma clang fp contract(off)
  const float var = sum * factor;
  const float v = var + eps;
  return (float)(1.0 / sqrt((double)v));
}

// four consecutive elements, kept as loaded
template <typename T> struct Raw4 { u32x2 v; };
template <> struct Raw4<float> { f32x4 v; };
template <typename T> __device__ __forceinline__ Raw4<T> load4(const T* p) {
  return Raw4<T>{*reinterpret_cast<const u32x2*>(p)};
}
template <> __device__ __forceinline__ Raw4<float> load4<float>(const float* p) {
  return Raw4<float>{*reinterpret_cast<const f32x4*>(p)};
}
template <typename T> __device__ __forceinline__ void unpack4(const Raw4<T>& r, float (&o)[4]);
template <> __device__ __forceinline__ void unpack4<bf16>(const Raw4<bf16>& r, float (&o)[4]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    o[2 * i] = __uint_as_float(r.v[i] << 16);
    o[2 * i + 1] = __uint_as_float(r.v[i] & 0xffff0000u);
  }
}
template <> __device__ __forceinline__ void unpack4<f16>(const Raw4<f16>& r, float (&o)[4]) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 h = __builtin_bit_cast(h4, r.v);
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (float)h[i];
}
template <> __device__ __forceinline__ void unpack4<float>(const Raw4<float>& r, float (&o)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = r.v[i];
}
template <typename T> __device__ __forceinline__ void store4(T* p, const float (&o)[4]);
template <> __device__ __forceinline__ void store4<bf16>(bf16* p, const float (&o)[4]) {
  *reinterpret_cast<u32x2*>(p) = u32x2{pack_bf2(o[0], o[1]), pack_bf2(o[2], o[3])};
}
template <> __device__ __forceinline__ void store4<f16>(f16* p, const float (&o)[4]) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const h4 h{(f16)o[0], (f16)o[1], (f16)o[2], (f16)o[3]};
  *reinterpret_cast<h4*>(p) = h;
}
template <> __device__ __forceinline__ void store4<float>(float* p, const float (&o)[4]) {
  *reinterpret_cast<f32x4*>(p) = f32x4{o[0], o[1], o[2], o[3]};
}

// y = w * T(x * r): the product rounded to fp32, then to T, then w * that
// rounded to T, as the module's operations.  The fp32 product is hidden from
// the optimiser: for fp16 it otherwise folds T(x * r) into one
// v_fma_mixlo_f16, which rounds the exact product to fp16 once and differs
// from the two roundings wherever they double-round.
template <typename T> __device__ __forceinline__ float primal(float w, float x, float r) {
#pragma clang fp contract(off)
  float p = x * r;
  asm("" : "+v"(p));
  return w * round_t<T>(p);
}

// Fast form, for rows torch reduces with bw <= 64 threads and no split: lane
// `sub` of a row is torch's thread x = sub, so the thread sums are formed in
// place and the shuffle tree is torch's.  64 / bw rows per wave.
//  VEC: the lane's loads are 4-element vectors x + k bw (width % 4 == 0); NV
//       bounds their number.  Otherwise (width < 128) the lane sums elements
//       sub and sub + bw, the only ones its loop reaches.
template <typename T, bool VEC, int NV>
__global__ __launch_bounds__(kThreads) void rmsnorm_fwd_lanes(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
    float* __restrict__ rstd, int64_t rows, int width, int bw, float factor, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int rows_per_wave = kWave / bw;
  const int64_t row = ((int64_t)blockIdx.x * (kThreads / kWave) + threadIdx.x / kWave) * rows_per_wave +
                      lane / bw;
  const int sub = lane & (bw - 1);
  const bool live = row < rows;
  const T* xr = x + (live ? row : 0) * width;
  float s;
  if constexpr (VEC) {
    const int nvec = width / 4;
    Raw4<T> v[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) v[k] = load4<T>(xr + min(sub + k * bw, nvec - 1) * 4);
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (sub + k * bw < nvec) {
        float f[4];
        unpack4<T>(v[k], f);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = add_rn(acc[i], sq_rn(f[i]));
      }
    }
    s = add_rn(add_rn(add_rn(acc[0], acc[1]), acc[2]), acc[3]);
    for (int off = 1; off < bw; off <<= 1) s = add_rn(s, __shfl_down(s, off, kWave));
    const float r = __shfl(torch_rstd(s, factor, eps), lane - sub, kWave);
    if (!live) return;
    if (sub == 0) rstd[row] = r;
    T* yr = y + row * width;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int vi = sub + k * bw;
      if (vi < nvec) {
        float f[4], wv[4], o[4];
        unpack4<T>(v[k], f);
        unpack4<T>(load4<T>(w + vi * 4), wv);
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = primal<T>(wv[i], f[i], r);
        store4<T>(yr + vi * 4, o);
      }
    }
  } else {
    const bool second = sub + bw < width;
    const float a = to_f(xr[sub]);
    const float b = to_f(xr[second ? sub + bw : sub]);
    s = add_rn(sq_rn(a), second ? sq_rn(b) : 0.f);
    for (int off = 1; off < bw; off <<= 1) s = add_rn(s, __shfl_down(s, off, kWave));
    const float r = __shfl(torch_rstd(s, factor, eps), lane - sub, kWave);
    if (!live) return;
    if (sub == 0) rstd[row] = r;
    T* yr = y + row * width;
    yr[sub] = from_f<T>(primal<T>(to_f(w[sub]), a, r));
    if (second) yr[sub + bw] = from_f<T>(primal<T>(to_f(w[sub + bw]), b, r));
  }
}

// General form: one wave per row for any RowReduce (more than 64 threads
// along the row for short row counts, split rows for wide ones, rows that
// start off a 16-byte boundary when width % 4 != 0).  Lane l forms the sums of
// torch threads l, l + 64, ... into LDS, then the trees run as torch's do.
constexpr int kMaxReduceThreads = 512;

template <typename T>
__global__ __launch_bounds__(kWave) void rmsnorm_fwd_rowwave(
    const T* __restrict__ x, const T* __restrict__ w, T* __restrict__ y,
    float* __restrict__ rstd, int64_t rows, int width, RowReduce c, float factor, float eps) {
  __shared__ float part[kMaxReduceThreads];
  __shared__ float ys[8];
  __shared__ float rs;
  const int lane = threadIdx.x;
  const int64_t row = blockIdx.x;
  const T* xr = x + row * width;
  const int nthreads = c.bw * c.bh;
  // torch's fp32 copy of the tensor starts 16-byte aligned, so row `row`
  // starts (row * width) % 4 elements past a boundary
  const int shift0 = c.vec ? (int)((row * (int64_t)width) & 3) : 0;
  auto sq_at = [&](int i) { return sq_rn(to_f(xr[i])); };
  for (int t = lane; t < nthreads; t += kWave) {
    const int tx = t % c.bw, ty = t / c.bw;
    const bool tail_ok = c.bh == 1 || ty == 0;  // should_reduce_tail
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    if (c.vec) {
      int end = width, d0 = 0, shift = shift0;
      if (shift > 0) {  // head of a row off the vector boundary
        d0 = -shift;
        end = width + shift;
        if (tx >= shift && tx < 4 && tail_ok) acc[0] = add_rn(0.f, sq_at(d0 + tx));
        end -= 4;
        d0 += 4;
      }
      for (int idx = tx + ty * c.ym; idx * 4 + 3 < end; idx += c.step)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = add_rn(acc[i], sq_at(d0 + idx * 4 + i));
      const int tail = end - end % 4 + tx;
      if (tail_ok && tail < end) acc[0] = add_rn(acc[0], sq_at(d0 + tail));
    } else {
      int idx = tx + ty * c.ym;
      for (; idx + 3 * c.step < width; idx += 4 * c.step)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = add_rn(acc[i], sq_at(idx + i * c.step));
      for (int i = 0; i < 4 && idx < width; ++i, idx += c.step) acc[i] = add_rn(acc[i], sq_at(idx));
    }
    part[t] = add_rn(add_rn(add_rn(acc[0], acc[1]), acc[2]), acc[3]);
  }
  __syncthreads();
  // block_x_reduce: LDS halving down to 64 threads per thread row
  for (int off = c.bw / 2; off >= kWave; off >>= 1) {
    for (int i = lane; i < c.bh * off; i += kWave) {
      const int tx = i % off, ty = i / off;
      part[ty * c.bw + tx] = add_rn(part[ty * c.bw + tx], part[ty * c.bw + tx + off]);
    }
    __syncthreads();
  }
  const int dim = min(c.bw, kWave);
  for (int ty = 0; ty < c.bh; ++ty) {
    float v = lane < dim ? part[ty * c.bw + lane] : 0.f;
    for (int off = 1; off < dim; off <<= 1) v = add_rn(v, __shfl_down(v, off, kWave));
    if (lane == 0) ys[ty] = v;
  }
  __syncthreads();
  if (lane == 0) {
    // block_y_reduce
    for (int off = c.bh / 2; off > 0; off >>= 1)
      for (int ty = 0; ty < off; ++ty) ys[ty] = add_rn(ys[ty], ys[ty + off]);
    const float r = torch_rstd(ys[0], factor, eps);
    rs = r;
    rstd[row] = r;
  }
  __syncthreads();
  const float r = rs;
  T* yr = y + row * width;
  for (int i = lane; i < width; i += kWave) yr[i] = from_f<T>(primal<T>(to_f(w[i]), to_f(xr[i]), r));
}

// ---------------------------------------------------------------------------
// backward, vector path.  Block b owns rows [b*slab, (b+1)*slab) and writes
// one fp32 partial dW row into part[b]; rmsnorm_dw_reduce sums the partials
// in a fixed order.
//
// The kernel streams x and dy once, so its speed is the number of row bytes
// in flight per CU.  Each wave owns one row (LPR = 64) or 64/LPR rows at a
// time and, when registers allow (BwdShape::kPrefetch), issues the loads of
// its next row before working on the current one.  Rows are held as loaded
// (Packed8) and unpacked twice -- once for dW and the row dot product, once
// for dx -- and w sits in LDS, so that two 8-wave blocks' worth of registers
// (<= 256 per lane) hold the prefetched row, the current row and the fp32 dW
// accumulators.
// ---------------------------------------------------------------------------
template <typename T, int NV, bool FULL> struct BwdShape {
  // prefetch where the compiled kernel then still fits 256 VGPRs unspilled
  static constexpr bool kPrefetch = NV <= 4 || (sizeof(T) == 2 && NV == 8 && FULL);
  static constexpr int kWaves = NV <= 8 ? 8 : 4;
  static constexpr int kThreads = kWaves * kWave;
};

template <typename T, int LPR, int NV, bool FULL>
__global__ __launch_bounds__((BwdShape<T, NV, FULL>::kThreads)) void rmsnorm_bwd_vec(
    const T* __restrict__ dy, const T* __restrict__ x, const T* __restrict__ w,
    const float* __restrict__ rstd, T* __restrict__ dx, float* __restrict__ part,
    int64_t rows, int width, int64_t slab, int want_dx, int want_dw) {
  using Shape = BwdShape<T, NV, FULL>;
  constexpr int kRowsPerWave = kWave / LPR;
  constexpr int kRowsPerPass = Shape::kWaves * kRowsPerWave;
  extern __shared__ float lds_dw[];  // [width] fp32 dW, then w as T [width]
  T* lds_w = reinterpret_cast<T*>(lds_dw + width);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int sub = lane % LPR;
  const int rsub = wave * kRowsPerWave + lane / LPR;  // 0 .. kRowsPerPass-1
  const int nvec = width / 8;
  const int64_t r0 = (int64_t)blockIdx.x * slab;
  const int64_t r1 = min(rows, r0 + slab);

  for (int v = threadIdx.x; v < nvec; v += Shape::kThreads)
    store_packed<T>(lds_w + v * 8, load_packed<T>(w + v * 8));

  // vector k of this lane: vi = sub + k*LPR; past the row end it reads the
  // row's last vector (in bounds) and is masked out
  auto col = [&](int k) { return FULL ? sub + k * LPR : min(sub + k * LPR, nvec - 1); };
  auto valid = [&](int k) { return FULL || sub + k * LPR < nvec; };
  auto load_row = [&](int64_t row, Packed8<T> (&xo)[NV], Packed8<T> (&go)[NV], float& ro) {
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      xo[k] = load_packed_once<T>(x + row * width + col(k) * 8);
      go[k] = load_packed_once<T>(dy + row * width + col(k) * 8);
    }
    ro = rstd[row];
  };

  float acc[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[k][i] = 0.f;
  const float inv_w = 1.f / (float)width;
  int64_t row = r0 + rsub;
  Packed8<T> xa[NV], ga[NV];
  float ra = 0.f;
  if (row < r1) load_row(row, xa, ga, ra);
  __syncthreads();  // lds_w
  for (; row < r1; row += kRowsPerPass) {
    const int64_t next = row + kRowsPerPass;
    Packed8<T> xb[NV], gb[NV];
    float rb = 0.f;
    if (Shape::kPrefetch && next < r1) load_row(next, xb, gb, rb);
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      if (valid(k)) {
        float xv[8], dv[8], wv[8];
        unpack<T>(xa[k], xv);
        unpack<T>(ga[k], dv);
        unpack<T>(load_packed<T>(lds_w + col(k) * 8), wv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc[k][i] = fmaf(dv[i] * xv[i], ra, acc[k][i]);
          dot = fmaf(dv[i] * wv[i], xv[i] * ra, dot);
        }
      }
    }
    // finish the first pass here: otherwise the optimiser sinks the dot
    // product into the dx branch and the dW update past it, keeping the
    // unpacked row live across the second pass
    asm volatile("" : "+v"(dot));
#pragma unroll
    for (int k = 0; k < NV; ++k)
      asm volatile("" : "+v"(acc[k][0]), "+v"(acc[k][1]), "+v"(acc[k][2]), "+v"(acc[k][3]),
                   "+v"(acc[k][4]), "+v"(acc[k][5]), "+v"(acc[k][6]), "+v"(acc[k][7]));
    if (want_dx) {
      dot = row_sum<LPR>(dot) * inv_w;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (valid(k)) {
          // recompute dy*w and xhat instead of keeping the first pass's
          // 16*NV products live across the row sum
          float xv[8], dv[8], wv[8], o[8];
          unpack<T>(opaque<T>(xa[k]), xv);
          unpack<T>(opaque<T>(ga[k]), dv);
          unpack<T>(opaque<T>(load_packed<T>(lds_w + col(k) * 8)), wv);
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = ra * (dv[i] * wv[i] - (xv[i] * ra) * dot);
          store8<T>(dx + row * width + col(k) * 8, o);
        }
      }
    }
    if (Shape::kPrefetch) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        xa[k] = xb[k];
        ga[k] = gb[k];
      }
      ra = rb;
    } else if (next < r1) {
      load_row(next, xa, ga, ra);
    }
  }
  if (!want_dw) return;
  // fixed-order combine of the block's row groups: group 0 stores, then each
  // later group adds in turn
  for (int g = 0; g < kRowsPerPass; ++g) {
    if (rsub == g) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (valid(k)) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            float* p = &lds_dw[col(k) * 8 + i];
            *p = (g == 0) ? acc[k][i] : (*p + acc[k][i]);
          }
        }
      }
    }
    __syncthreads();
  }
  for (int c = threadIdx.x; c < width; c += Shape::kThreads)
    part[(int64_t)blockIdx.x * width + c] = lds_dw[c];
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

// dW = T(sum over partial rows in a fixed order).  A block owns 64 columns
// (one per lane, so each load is a 256-byte row piece); its 16 waves each sum
// a contiguous run of partial rows, sixteen independent loads at a time, and
// wave 0 adds the 16 wave sums in wave order.
constexpr int kReduceWaves = 16;

template <typename T>
__global__ __launch_bounds__(kReduceWaves * kWave) void rmsnorm_dw_reduce(
    const float* __restrict__ part, T* __restrict__ dw, int nparts, int width) {
  __shared__ float red[kReduceWaves][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int c = blockIdx.x * kWave + lane;
  const int cc = min(c, width - 1);
  const int per = (nparts + kReduceWaves - 1) / kReduceWaves;
  const int p0 = min(nparts, wave * per);
  const int p1 = min(nparts, p0 + per);
  float s = 0.f;
  int p = p0;
  for (; p + 16 <= p1; p += 16) {
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) v[j] = part[(int64_t)(p + j) * width + cc];
#pragma unroll
    for (int j = 0; j < 16; ++j) s += v[j];
  }
  for (; p < p1; ++p) s += part[(int64_t)p * width + cc];
  red[wave][lane] = s;
  __syncthreads();
  if (wave != 0 || c >= width) return;
  float t = red[0][lane];
#pragma unroll
  for (int q = 1; q < kReduceWaves; ++q) t += red[q][lane];
  dw[c] = from_f<T>(t);
}

// dW of zero rows
template <typename T>
__global__ __launch_bounds__(kThreads) void zero_fill(T* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) out[i] = from_f<T>(0.f);
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

int64_t bwd_parts(int64_t rows, int64_t width) {
  // at least 32 rows per block, so the partial rows (written and read once)
  // stay within 8/(6*32) of the kernel's traffic; at most 256 blocks for rows
  // of 2048 and more elements -- one 8-wave block per CU is enough bytes in
  // flight there -- and up to 1024 for narrower rows, whose blocks carry less
  int64_t parts = (rows + 31) / 32;
  const int64_t max_parts = width >= 2048 ? 256 : 1024;
  if (parts > max_parts) parts = max_parts;
  if (parts < 1) parts = 1;
  return parts;
}

// CU count of the device a stream belongs to (torch's schedule consults it)
int stream_cus(hipStream_t s) {
  int dev = 0;
  if (s == nullptr || hipStreamGetDevice(s, &dev) != hipSuccess) (void)hipGetDevice(&dev);
  static int cached[64] = {0};
  if (dev >= 0 && dev < 64 && cached[dev] > 0) return cached[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 256;
  if (dev >= 0 && dev < 64) cached[dev] = n;
  return n;
}

template <typename T>
int launch_fwd(const void* x, const void* w, void* y, float* rstd, int64_t rows, int width,
               float eps, hipStream_t s) {
  RowReduce c;
  if (!torch_row_reduce(rows, width, stream_cus(s), c)) {
    set_error("ts_rmsnorm_fwd: a single row of width %d is summed across work-groups by torch; "
              "that order is not reproduced", width);
    return TS_ERR_INVALID;
  }
  // MeanOps' factor: float(outputs) / numel, the division in float
  const float factor = (float)rows / (float)(rows * (int64_t)width);
  if (c.bh == 1 && c.bw <= kWave && (!c.vec || width % 4 == 0)) {
    const int64_t rows_per_block = (kThreads / kWave) * (kWave / c.bw);
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block));
    ts::TimedLaunch timed_("rmsnorm.rmsnorm_fwd_lanes", s);
    if (!c.vec) {
      hipLaunchKernelGGL((rmsnorm_fwd_lanes<T, false, 1>), grid, dim3(kThreads), 0, s, (const T*)x,
                         (const T*)w, (T*)y, rstd, rows, width, c.bw, factor, eps);
      return check_launch("ts_rmsnorm_fwd");
    }
    const int loads = (width / 4 + c.bw - 1) / c.bw;
#define TS_FWD(NV)                                                                             \
  if (loads <= NV) {                                                                           \
    hipLaunchKernelGGL((rmsnorm_fwd_lanes<T, true, NV>), grid, dim3(kThreads), 0, s,           \
                       (const T*)x, (const T*)w, (T*)y, rstd, rows, width, c.bw, factor, eps); \
    return check_launch("ts_rmsnorm_fwd");                                                     \
  }
    TS_FWD(1) TS_FWD(2) TS_FWD(4) TS_FWD(8) TS_FWD(16) TS_FWD(32)
#undef TS_FWD
  }
  if (rows > 0x7fffffff) {
    set_error("ts_rmsnorm_fwd: %lld rows exceed one launch", (long long)rows);
    return TS_ERR_INVALID;
  }
  ts::TimedLaunch timed_("rmsnorm.rmsnorm_fwd_rowwave", s);
  hipLaunchKernelGGL(rmsnorm_fwd_rowwave<T>, dim3((unsigned)rows), dim3(kWave), 0, s, (const T*)x,
                     (const T*)w, (T*)y, rstd, rows, width, c, factor, eps);
  return check_launch("ts_rmsnorm_fwd");
}

template <typename T>
int launch_bwd(const void* dy, const void* x, const void* w, const float* rstd, void* dx,
               void* dw, float* part, int64_t rows, int width, hipStream_t s) {
  const Geometry g = pick(width, 0);
  const int64_t parts = bwd_parts(rows, width);
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
    // LDS: the fp32 dW row, then w as T
    const size_t lds = (size_t)width * (sizeof(float) + sizeof(T));
    const dim3 grid((unsigned)parts);
    const bool full = width == 8 * g.lpr * g.nv;
    bool launched = false;
#define TS_BWD(LPR, NV)                                                                      \
  if (!launched && g.lpr == LPR && g.nv == NV) {                                             \
    ts::TimedLaunch timed_("rmsnorm.rmsnorm_bwd_vec", s);                                    \
    if (full)                                                                                \
      hipLaunchKernelGGL((rmsnorm_bwd_vec<T, LPR, NV, true>), grid,                          \
                         dim3(BwdShape<T, NV, true>::kThreads), lds, s,                      \
                         (const T*)dy, (const T*)x, (const T*)w, rstd, (T*)dx, part, rows,   \
                         width, slab, want_dx, want_dw);                                     \
    else                                                                                     \
      hipLaunchKernelGGL((rmsnorm_bwd_vec<T, LPR, NV, false>), grid,                         \
                         dim3(BwdShape<T, NV, false>::kThreads), lds, s,                     \
                         (const T*)dy, (const T*)x, (const T*)w, rstd, (T*)dx, part, rows,   \
                         width, slab, want_dx, want_dw);                                     \
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
  { ts::TimedLaunch timed_("rmsnorm.rmsnorm_dw_reduce", s); hipLaunchKernelGGL(rmsnorm_dw_reduce<T>, dim3((unsigned)((width + kWave - 1) / kWave)),
                     dim3(kReduceWaves * kWave), 0, s, (const float*)part, (T*)dw, (int)parts, width); }
  return check_launch("ts_rmsnorm_bwd (dW reduce)");
}

template <typename T>
int launch_zero(void* out, int64_t n, hipStream_t s) {
  hipLaunchKernelGGL(zero_fill<T>, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                     (T*)out, n);
  return check_launch("ts_rmsnorm_bwd (zero dW)");
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

int ts_rmsnorm_supported(int64_t rows, int64_t width, void* stream) {
  if (rows < 0 || width <= 0 || width > (1 << 24)) return 0;
  if (rows > 0) {
    ts::RowReduce c;
    if (!ts::torch_row_reduce(rows, width, ts::stream_cus((hipStream_t)stream), c)) return 0;
    const bool lanes = c.bh == 1 && c.bw <= ts::kWave && (!c.vec || width % 4 == 0);
    if (!lanes && rows > 0x7fffffff) return 0;
  }
  const ts::Geometry g = ts::pick(width, 0);
  if (g.lpr == 0 && (width + 4) * (int64_t)sizeof(float) > 160 * 1024) return 0;
  return 1;
}

int64_t ts_rmsnorm_bwd_workspace(int64_t rows, int64_t width) {
  if (rows <= 0 || width <= 0) return 0;
  return ts::bwd_parts(rows, width) * width * (int64_t)sizeof(float);
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
    // a fill kernel rather than a memset node, so the call can be captured
    if (!dw) return TS_OK;
    switch (dtype) {
      case TS_BF16: return ts::launch_zero<ts::bf16>(dw, width, s);
      case TS_F16: return ts::launch_zero<ts::f16>(dw, width, s);
      case TS_F32: return ts::launch_zero<float>(dw, width, s);
    }
    ts::set_error("ts_rmsnorm_bwd: unsupported dtype code %d", dtype);
    return TS_ERR_INVALID;
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
