// Fused chunked-vocab logprob / entropy at the inputs' own precision (fp32 or
// fp64 hidden states and head): logits, softmax statistics, dlogits and the
// two VJP products all in that type, as the reference keeps FP32/FP64 inputs
// at their precision (accel/fused_logprob.py:27-58, `_accum_dtype`: only
// bf16/fp16 widen).  The bf16/fp16 operators run on MFMA (logprob.hip);
// these take the vector ALUs, which give fp32 and fp64 FMAs with no operand
// rounding.
//
// One tile product serves every kernel: a 256-thread work-group forms a
// 64 x 64 tile of C(m, n) = sum_k A(m, k) B(k, n) over operands given by
// element strides (a K-contiguous and an M-contiguous operand are both read
// with consecutive threads on consecutive addresses), staging 16-deep K
// slices through LDS; thread (ty, tx) = (tid / 16, tid % 16) owns rows
// 4 ty .. 4 ty + 3 and columns 4 tx .. 4 tx + 3.  The 16 threads sharing a
// row are 16 consecutive lanes of one wave, so row reductions of a tile are
// xor-shuffles within the wave.
//
//   forward   a work-group walks the vocabulary tiles vg, vg + G, ... of its
//             64 rows (G groups), merging per row (max, sum exp(l - max),
//             sum exp(l - max) (l - max)) in registers, and writes one partial
//             per group; a combine kernel (one wave per row) merges the G
//             partials into lse and entropy and takes the target logit as a
//             dot product of the row with the target's weight row.
//   backward  the same tile product recomputes a block of logits and writes
//             dlogits = -p (g_lp + g_H (log p + H)) + g_lp [v == t] in the
//             input type; grad_hidden = dlogits . W and grad_weight +=
//             dlogits^T . hidden are two more tile products.
#include <cmath>

#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace lpx {

constexpr int BT = 64;        // tile rows and columns
constexpr int BKX = 16;       // K per LDS slice
constexpr int kThreads = 256;
constexpr int kMaxGroups = 64;  // vocabulary groups of the forward (partials per row)

template <typename T> __device__ __forceinline__ T inf_of() { return (T)__builtin_huge_val(); }
__device__ __forceinline__ float exp_of(float x) { return expf(x); }
__device__ __forceinline__ double exp_of(double x) { return exp(x); }
__device__ __forceinline__ float log_of(float x) { return logf(x); }
__device__ __forceinline__ double log_of(double x) { return log(x); }

// C tile (m0, n0) of sum_k A(m, k) B(k, n) into acc[i][j] (row 4 ty + i,
// column 4 tx + j); A(m, k) = a[m a_m + k a_k], B(k, n) = b[k b_k + n b_n];
// elements past M, N or K read as zero.
template <typename T>
__device__ __forceinline__ void tile_product(const T* __restrict__ a, int64_t a_m, int64_t a_k,
                                             const T* __restrict__ b, int64_t b_k, int64_t b_n, int64_t M,
                                             int64_t N, int64_t K, int64_t m0, int64_t n0, T (*as)[BT + 1],
                                             T (*bs)[BT + 1], T acc[4][4]) {
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (T)0;
  const bool a_kfast = a_k == 1, b_kfast = b_k == 1;
  for (int64_t k0 = 0; k0 < K; k0 += BKX) {
    // 16 x 64 elements of each operand, four per thread, the operand's
    // contiguous index fastest over consecutive threads
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = tid + kThreads * r;
      const int mm = a_kfast ? e / BKX : e % BT;
      const int kk = a_kfast ? e % BKX : e / BT;
      const int64_t m = m0 + mm, k = k0 + kk;
      as[kk][mm] = (m < M && k < K) ? a[m * a_m + k * a_k] : (T)0;
      const int nn = b_kfast ? e / BKX : e % BT;
      const int kb = b_kfast ? e % BKX : e / BT;
      const int64_t n = n0 + nn, kq = k0 + kb;
      bs[kb][nn] = (n < N && kq < K) ? b[kq * b_k + n * b_n] : (T)0;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BKX; ++kk) {
      T av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = as[kk][4 * ty + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = bs[kk][4 * tx + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fma(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
}

// (max, sum exp(l - max), sum exp(l - max) (l - max)) of two disjoint sets of
// logits, either of which may be empty (max = -inf)
template <typename T>
__device__ __forceinline__ void merge_stats(T& m, T& s, T& e, T mo, T so, T eo) {
  if (mo == -inf_of<T>()) return;
  if (m == -inf_of<T>()) {
    m = mo;
    s = so;
    e = eo;
    return;
  }
  const T mn = m > mo ? m : mo;
  const T ca = exp_of(m - mn), cb = exp_of(mo - mn);
  e = ca * (e + s * (m - mn)) + cb * (eo + so * (mo - mn));
  s = ca * s + cb * so;
  m = mn;
}

template <typename T>
__device__ __forceinline__ T shfl_x(T v, int mask) {
  return __shfl_xor(v, mask, 64);
}

// partial[(g * 3 + c) * rows + r]: row r's statistics c (max, sum, sum
// (l - max)) over the vocabulary tiles g, g + G, ...
template <typename T>
__global__ __launch_bounds__(kThreads) void fwd_stats_kernel(const T* __restrict__ h, int64_t ld_h,
                                                             const T* __restrict__ w, int64_t ld_w, int64_t rows,
                                                             int64_t dim, int64_t vocab, int groups,
                                                             T* __restrict__ partial) {
  __shared__ T as[BKX][BT + 1];
  __shared__ T bs[BKX][BT + 1];
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int g = blockIdx.x % groups;
  const int64_t m0 = (int64_t)(blockIdx.x / groups) * BT;
  const int64_t n_tiles = (vocab + BT - 1) / BT;
  T sm[4], ss[4], se[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    sm[i] = -inf_of<T>();
    ss[i] = (T)0;
    se[i] = (T)0;
  }
  for (int64_t vt = g; vt < n_tiles; vt += groups) {
    T acc[4][4];
    // logits (row m, vocab n): A = hidden rows (K-contiguous), B(k, n) = w[n][k]
    tile_product<T>(h, ld_h, 1, w, 1, ld_w, rows, vocab, dim, m0, vt * BT, as, bs, acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      T mx = -inf_of<T>();
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (vt * BT + 4 * tx + j < vocab) mx = acc[i][j] > mx ? acc[i][j] : mx;
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        const T y = shfl_x(mx, o);
        mx = y > mx ? y : mx;
      }
      T s = (T)0, e = (T)0;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (vt * BT + 4 * tx + j < vocab) {
          const T x = acc[i][j] - mx;
          const T p = exp_of(x);
          s += p;
          e += p * x;
        }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        s += shfl_x(s, o);
        e += shfl_x(e, o);
      }
      merge_stats(sm[i], ss[i], se[i], mx, s, e);
    }
  }
  if (tx == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t r = m0 + 4 * ty + i;
      if (r < rows) {
        partial[(3 * (int64_t)g + 0) * rows + r] = sm[i];
        partial[(3 * (int64_t)g + 1) * rows + r] = ss[i];
        partial[(3 * (int64_t)g + 2) * rows + r] = se[i];
      }
    }
  }
}

// one wave per row: merge the G partials, then the target logit as a dot
// product; logprob = l_t - lse (NaN for a target outside the vocabulary),
// entropy = log S - E / S
template <typename T>
__global__ __launch_bounds__(kThreads) void combine_kernel(const T* __restrict__ partial, int groups,
                                                           const T* __restrict__ h, int64_t ld_h,
                                                           const T* __restrict__ w, int64_t ld_w,
                                                           const int64_t* __restrict__ target, int64_t rows,
                                                           int64_t dim, int64_t vocab, T* __restrict__ logprob,
                                                           T* __restrict__ entropy, T* __restrict__ lse) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (r >= rows) return;
  T m = -inf_of<T>(), s = (T)0, e = (T)0;
  for (int g = lane; g < groups; g += 64)
    merge_stats(m, s, e, partial[(3 * (int64_t)g + 0) * rows + r], partial[(3 * (int64_t)g + 1) * rows + r],
                partial[(3 * (int64_t)g + 2) * rows + r]);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const T mo = shfl_x(m, o), so = shfl_x(s, o), eo = shfl_x(e, o);
    merge_stats(m, s, e, mo, so, eo);
  }
  const int64_t t = target[r];
  const bool valid = t >= 0 && t < vocab;
  T dot = (T)0;
  if (valid)
    for (int64_t d = lane; d < dim; d += 64) dot = fma(h[r * ld_h + d], w[t * ld_w + d], dot);
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) dot += shfl_x(dot, o);
  if (lane == 0) {
    const T l = m + log_of(s);
    lse[r] = l;
    logprob[r] = valid ? dot - l : (T)__builtin_nan("");
    if (entropy) entropy[r] = log_of(s) - e / s;
  }
}

// dlogits block [rows, vocab] (row stride ld_dl): -p (g_lp + g_H (log p + H))
// + g_lp [v == t], p = exp(l - lse); g_ent NULL: the logprob-only objective
template <typename T>
__global__ __launch_bounds__(kThreads) void dlogits_kernel(const T* __restrict__ h, int64_t ld_h,
                                                           const T* __restrict__ w, int64_t ld_w,
                                                           const int64_t* __restrict__ target,
                                                           const T* __restrict__ lse, const T* __restrict__ ent,
                                                           const T* __restrict__ g_lp, const T* __restrict__ g_ent,
                                                           int64_t rows, int64_t dim, int64_t vocab,
                                                           T* __restrict__ dl, int64_t ld_dl, int64_t n_vtiles) {
  __shared__ T as[BKX][BT + 1];
  __shared__ T bs[BKX][BT + 1];
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int64_t vt = blockIdx.x % n_vtiles;
  const int64_t m0 = (int64_t)(blockIdx.x / n_vtiles) * BT, n0 = vt * BT;
  T acc[4][4];
  tile_product<T>(h, ld_h, 1, w, 1, ld_w, rows, vocab, dim, m0, n0, as, bs, acc);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = m0 + 4 * ty + i;
    if (r >= rows) continue;
    const T l0 = lse[r], g = g_lp[r];
    const T ge = g_ent ? g_ent[r] : (T)0, hr = g_ent ? ent[r] : (T)0;
    const int64_t t = target[r];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t v = n0 + 4 * tx + j;
      if (v >= vocab) continue;
      const T lp = acc[i][j] - l0;  // log p
      const T p = exp_of(lp);
      T d = -p * (g_ent ? g + ge * (lp + hr) : g);
      if (v == t) d += g;
      dl[r * ld_dl + v] = d;
    }
  }
}

// C [M, N] (row stride ldc) = (or +=) A . B
template <typename T>
__global__ __launch_bounds__(kThreads) void matmul_kernel(const T* __restrict__ a, int64_t a_m, int64_t a_k,
                                                          const T* __restrict__ b, int64_t b_k, int64_t b_n,
                                                          int64_t M, int64_t N, int64_t K, T* __restrict__ c,
                                                          int64_t ldc, int accumulate, int64_t n_tiles) {
  __shared__ T as[BKX][BT + 1];
  __shared__ T bs[BKX][BT + 1];
  const int tid = threadIdx.x, ty = tid >> 4, tx = tid & 15;
  const int64_t m0 = (int64_t)(blockIdx.x / n_tiles) * BT, n0 = (int64_t)(blockIdx.x % n_tiles) * BT;
  T acc[4][4];
  tile_product<T>(a, a_m, a_k, b, b_k, b_n, M, N, K, m0, n0, as, bs, acc);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t m = m0 + 4 * ty + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t n = n0 + 4 * tx + j;
      if (n >= N) continue;
      T* p = c + m * ldc + n;
      *p = accumulate ? *p + acc[i][j] : acc[i][j];
    }
  }
}

int groups_of(int64_t vocab) {
  const int64_t tiles = (vocab + BT - 1) / BT;
  return (int)std::min<int64_t>(tiles, kMaxGroups);
}

int elem_bytes(int dtype) { return dtype == TS_F64 ? 8 : 4; }

template <typename T>
int fwd_t(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w, const int64_t* target, int64_t rows,
          int64_t dim, int64_t vocab, void* logprob, void* entropy, void* lse, void* workspace, hipStream_t s) {
  const int groups = groups_of(vocab);
  const int64_t row_tiles = (rows + BT - 1) / BT;
  {
    ts::TimedLaunch timed_("logprob.exact_fwd_stats_kernel", s);
    hipLaunchKernelGGL(fwd_stats_kernel<T>, dim3((unsigned)(row_tiles * groups)), dim3(kThreads), 0, s,
                       (const T*)hidden, ld_h, (const T*)weight, ld_w, rows, dim, vocab, groups, (T*)workspace);
  }
  {
    ts::TimedLaunch timed_("logprob.exact_combine_kernel", s);
    hipLaunchKernelGGL(combine_kernel<T>, dim3((unsigned)((rows + 3) / 4)), dim3(kThreads), 0, s,
                       (const T*)workspace, groups, (const T*)hidden, ld_h, (const T*)weight, ld_w, target, rows,
                       dim, vocab, (T*)logprob, (T*)entropy, (T*)lse);
  }
  return ts::check_launch("ts_logprob_fwd_exact");
}

template <typename T>
int dlogits_t(const void* hidden, int64_t ld_h, const void* weight, int64_t ld_w, const int64_t* target,
              const void* lse, const void* ent, const void* g_lp, const void* g_ent, int64_t rows, int64_t dim,
              int64_t vocab, void* dl, int64_t ld_dl, hipStream_t s) {
  const int64_t n_vtiles = (vocab + BT - 1) / BT, row_tiles = (rows + BT - 1) / BT;
  ts::TimedLaunch timed_("logprob.exact_dlogits_kernel", s);
  hipLaunchKernelGGL(dlogits_kernel<T>, dim3((unsigned)(row_tiles * n_vtiles)), dim3(kThreads), 0, s,
                     (const T*)hidden, ld_h, (const T*)weight, ld_w, target, (const T*)lse, (const T*)ent,
                     (const T*)g_lp, (const T*)g_ent, rows, dim, vocab, (T*)dl, ld_dl, n_vtiles);
  return ts::check_launch("ts_logprob_dlogits_exact");
}

template <typename T>
int matmul_t(const void* a, int64_t a_m, int64_t a_k, const void* b, int64_t b_k, int64_t b_n, int64_t m,
             int64_t n, int64_t k, void* c, int64_t ldc, int accumulate, hipStream_t s) {
  const int64_t n_tiles = (n + BT - 1) / BT, m_tiles = (m + BT - 1) / BT;
  ts::TimedLaunch timed_("logprob.exact_matmul_kernel", s);
  hipLaunchKernelGGL(matmul_kernel<T>, dim3((unsigned)(m_tiles * n_tiles)), dim3(kThreads), 0, s, (const T*)a,
                     a_m, a_k, (const T*)b, b_k, b_n, m, n, k, (T*)c, ldc, accumulate, n_tiles);
  return ts::check_launch("ts_matmul_exact");
}

}  // namespace lpx
}  // namespace ts

using namespace ts::lpx;

extern "C" {

int64_t ts_logprob_fwd_exact_workspace(int64_t rows, int64_t vocab, int dtype) {
  if (rows < 0 || vocab < 1 || (dtype != TS_F32 && dtype != TS_F64)) return -1;
  return 3 * (int64_t)groups_of(vocab) * rows * elem_bytes(dtype);
}

int ts_logprob_fwd_exact(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                         const int64_t* target, int64_t rows, int64_t dim, int64_t vocab, void* logprob,
                         void* entropy, void* lse, void* workspace, int64_t workspace_bytes, int dtype,
                         void* stream) {
  TS_CHECK_ARG(dtype == TS_F32 || dtype == TS_F64, "ts_logprob_fwd_exact: dtype must be TS_F32 or TS_F64");
  TS_CHECK_ARG(rows >= 0 && dim >= 1 && vocab >= 1, "ts_logprob_fwd_exact: rows >= 0, dim >= 1, vocab >= 1");
  TS_CHECK_ARG(ld_hidden >= dim && ld_weight >= dim, "ts_logprob_fwd_exact: leading dimensions below dim");
  TS_CHECK_ARG((rows + 3) / 4 < (int64_t)1 << 31 && ((rows + BT - 1) / BT) * groups_of(vocab) < (int64_t)1 << 31,
               "ts_logprob_fwd_exact: too many rows for one launch");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(hidden && weight && target && logprob && lse && workspace,
               "ts_logprob_fwd_exact: null pointer");
  TS_CHECK_ARG(workspace_bytes >= ts_logprob_fwd_exact_workspace(rows, vocab, dtype),
               "ts_logprob_fwd_exact: workspace too small");
  hipStream_t s = (hipStream_t)stream;
  return dtype == TS_F64 ? fwd_t<double>(hidden, ld_hidden, weight, ld_weight, target, rows, dim, vocab, logprob,
                                         entropy, lse, workspace, s)
                         : fwd_t<float>(hidden, ld_hidden, weight, ld_weight, target, rows, dim, vocab, logprob,
                                        entropy, lse, workspace, s);
}

int ts_logprob_dlogits_exact(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                             const int64_t* target, const void* lse, const void* entropy, const void* grad_lp,
                             const void* grad_ent, int64_t rows, int64_t dim, int64_t vocab, void* dlogits,
                             int64_t ld_dlogits, int dtype, void* stream) {
  TS_CHECK_ARG(dtype == TS_F32 || dtype == TS_F64, "ts_logprob_dlogits_exact: dtype must be TS_F32 or TS_F64");
  TS_CHECK_ARG(rows >= 0 && dim >= 1 && vocab >= 1, "ts_logprob_dlogits_exact: rows >= 0, dim >= 1, vocab >= 1");
  TS_CHECK_ARG(ld_hidden >= dim && ld_weight >= dim && ld_dlogits >= vocab,
               "ts_logprob_dlogits_exact: leading dimensions too small");
  TS_CHECK_ARG(!grad_ent || entropy, "ts_logprob_dlogits_exact: grad_ent needs entropy");
  TS_CHECK_ARG(((rows + BT - 1) / BT) * ((vocab + BT - 1) / BT) < (int64_t)1 << 31,
               "ts_logprob_dlogits_exact: block too large for one launch");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(hidden && weight && target && lse && grad_lp && dlogits, "ts_logprob_dlogits_exact: null pointer");
  hipStream_t s = (hipStream_t)stream;
  return dtype == TS_F64 ? dlogits_t<double>(hidden, ld_hidden, weight, ld_weight, target, lse, entropy, grad_lp,
                                             grad_ent, rows, dim, vocab, dlogits, ld_dlogits, s)
                         : dlogits_t<float>(hidden, ld_hidden, weight, ld_weight, target, lse, entropy, grad_lp,
                                            grad_ent, rows, dim, vocab, dlogits, ld_dlogits, s);
}

int ts_matmul_exact(const void* a, int64_t a_m, int64_t a_k, const void* b, int64_t b_k, int64_t b_n, int64_t m,
                    int64_t n, int64_t k, void* c, int64_t ldc, int accumulate, int dtype, void* stream) {
  TS_CHECK_ARG(dtype == TS_F32 || dtype == TS_F64, "ts_matmul_exact: dtype must be TS_F32 or TS_F64");
  TS_CHECK_ARG(m >= 0 && n >= 0 && k >= 0 && ldc >= n, "ts_matmul_exact: bad shape");
  TS_CHECK_ARG(((m + BT - 1) / BT) * ((n + BT - 1) / BT) < (int64_t)1 << 31, "ts_matmul_exact: too large");
  if (m == 0 || n == 0) return TS_OK;
  TS_CHECK_ARG(c && (k == 0 || (a && b)), "ts_matmul_exact: null pointer");
  hipStream_t s = (hipStream_t)stream;
  return dtype == TS_F64 ? matmul_t<double>(a, a_m, a_k, b, b_k, b_n, m, n, k, c, ldc, accumulate, s)
                         : matmul_t<float>(a, a_m, a_k, b, b_k, b_n, m, n, k, c, ldc, accumulate, s);
}

}  // extern "C"
