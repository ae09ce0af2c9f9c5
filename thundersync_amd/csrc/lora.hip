// Merged-weight LoRA linear for gfx950 (bf16 or fp16 operands, fp32 accumulation).
//
// Reference: accel/fused_lora.py:26-48 (FusedLoRALinear).  The adapters are
// merged into the base weight by the caller (W_eff = W + s B A), so the
// forward is one GEMM; the backward is the exact derivative of the unmerged
// expression:
//
//   grad_x = g W_eff                       (g: grad_out [rows, out])
//   grad_A = s (g B)^T x   = s u^T x       u = g B   [rows, rank]
//   grad_B = s g^T (x A^T) = s g^T t       t = x A^T [rows, rank]
//
// Every product runs on the 256 x 256 MFMA tile of gemm_core.h:
//   forward       y^T tile = W_tile . x_tile^T, staged through LDS into
//                 coalesced 16-byte row stores of y;
//   grad_x        the logprob grad-hidden kernel (dlogits . W with W read in
//                 place as the K-strided operand), g in the role of dlogits;
//   rank          u^T and t^T ([rank, rows], bf16, zero past the last row) in
//                 one launch: C = A_op . B_op^T with A_op the row tile of g
//                 (or x) and B_op = B^T (or A), both K-contiguous;
//   adapter       grad_A^T / grad_B partial sums over fixed row ranges of the
//                 contraction (rows), one launch each, C = u^T . x^T-tile
//                 (x K-strided) and C = g^T-tile . t (g K-strided);
//   reduce        sums the row ranges in range order and scales by s.
// The rank-sized side of a rank/adapter tile holds `rank` valid rows of 256:
// those products are bound by reading g and x (twice each over the backward),
// not by the MFMA work the tile leaves idle.
#include <algorithm>

#include "common.h"
#include "gemm_core.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace lora {

using namespace ts::gemm;

constexpr int kThreads = 256;
constexpr int OPITCH = TM + 8;  // staging pitch (bf16) of [64 rows][TM columns] quarter tiles
static_assert(64 * OPITCH <= kStageElems + 1024, "a quarter of the output tile fits one ring stage");

// ---------------------------------------------------------------------------
// forward: y[m][n] = sum_k x[m][k] W[n][k]
// ---------------------------------------------------------------------------
struct FwdArgs {
  const bf16* x;
  int64_t ldx;
  const bf16* w;
  int64_t ldw;
  int rows, in, out;
  int n_mtiles, n_ntiles;
  bf16* y;
  int64_t ldy;
};

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void lora_fwd_kernel(FwdArgs p) {
  GEMM_RING
  const int total = p.n_mtiles * p.n_ntiles;
  int nt, mt;
  grouped_tile(xcd_logical(blockIdx.x, total), p.n_ntiles, p.n_mtiles, nt, mt);
  const int n0 = nt * TM, m0 = mt * TN;
  f32x16 acc[4][NI];
  gemm_tile<E, false, false>(acc, p.w + (int64_t)n0 * p.ldw, p.ldw, min(TM, p.out - n0),
                          p.x + (int64_t)m0 * p.ldx, p.ldx, min(TN, p.rows - m0), p.in, s0, s1, s2, s3);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  // rows 64 q .. 64 q + 63 of the tile are staged in ring stage q as [64][OPITCH]
  auto quarter = [&](int q) -> bf16* { return q == 0 ? s0 : q == 1 ? s1 : q == 2 ? s2 : s3; };
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = b_row(ni, lane, wn);  // row of x / y within the tile
    bf16* o = quarter(col >> 6) + (col & 63) * OPITCH;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const f32x16& a = acc[mi][ni];
        // output columns a_row(mi, 4 i4 .. 4 i4 + 3) are consecutive: one 8-byte write
        *reinterpret_cast<u32x2*>(o + a_row(mi, 4 * i4, lane, wm)) =
            u32x2{pack2<E>(a[4 * i4], a[4 * i4 + 1]), pack2<E>(a[4 * i4 + 2], a[4 * i4 + 3])};
      }
  }
  __syncthreads();
  const int nmax = min(TM, p.out - n0);  // a multiple of 8
#pragma unroll 4
  for (int it = 0; it < (TN * TM / 8) / kGemmThreads; ++it) {
    const int c = it * kGemmThreads + tid;
    const int row = c / (TM / 8), chunk = (c % (TM / 8)) * 8;
    const int m = m0 + row;
    if (m < p.rows && chunk < nmax)
      *reinterpret_cast<u32x4*>(p.y + (int64_t)m * p.ldy + n0 + chunk) =
          *reinterpret_cast<const u32x4*>(quarter(row >> 6) + (row & 63) * OPITCH + chunk);
  }
}

// ---------------------------------------------------------------------------
// rank projections: out^T[r][m] = sum_k src[m][k] proj[r][k], for
// (src, proj) = (g, B^T) -> u^T and (x, A) -> t^T, in one launch
// ---------------------------------------------------------------------------
struct RankJob {
  const bf16* src;  // [rows][ld_src]
  int64_t ld_src;
  const bf16* proj;  // [rank][ld_proj]
  int64_t ld_proj;
  int k;             // contraction length
  bf16* out;         // [rank][ld_out]
};

struct RankArgs {
  RankJob job[2];
  int n_jobs;
  int rows, rank, n_mtiles;
  int64_t ld_out;  // rows rounded up to a multiple of 8; columns rows .. ld_out - 1 are written as zeros
};

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void lora_rank_kernel(RankArgs p) {
  GEMM_RING
  const int id = xcd_logical(blockIdx.x, p.n_mtiles * p.n_jobs);
  const int j = id / p.n_mtiles;
  const RankJob& job = p.job[j];
  const int m0 = (id - j * p.n_mtiles) * TM;
  f32x16 acc[4][NI];
  gemm_tile<E, false, false>(acc, job.src + (int64_t)m0 * job.ld_src, job.ld_src, min(TM, p.rows - m0), job.proj,
                          job.ld_proj, p.rank, job.k, s0, s1, s2, s3);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  // rows past `rows` came in as zeros, so their sums are exact zeros: the
  // padding columns of out^T are written from them
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int r = b_row(ni, lane, wn);
    if (r >= p.rank) continue;
    bf16* o = job.out + (int64_t)r * p.ld_out;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int m = m0 + a_row(mi, 4 * i4, lane, wm);
        const f32x16& a = acc[mi][ni];
        if (m + 3 < p.ld_out)
          *reinterpret_cast<u32x2*>(o + m) =
              u32x2{pack2<E>(a[4 * i4], a[4 * i4 + 1]), pack2<E>(a[4 * i4 + 2], a[4 * i4 + 3])};
      }
  }
}

// ---------------------------------------------------------------------------
// adapter gradients, partial sums over the row range [kb, kb + kper) of split s:
//   A side: part_a[s][r][k] = sum_m u^T[r][m] x[m][k]   (tile over k)
//   B side: part_b[s][n][r] = sum_m g[m][n] t^T[r][m]   (tile over n)
// ---------------------------------------------------------------------------
struct AdapterArgs {
  const bf16* uT;   // [rank][ld_rt]   (A side) or t^T (B side)
  int64_t ld_rt;
  const bf16* big;  // x [rows][ld_big] (A side) or g (B side)
  int64_t ld_big;
  int rows, rank, width;  // width: in_features (A side) or out_features (B side)
  int n_tiles, msplit, kper;
  float* part;      // A side [msplit][rank][width]; B side [msplit][width][rank]
};

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void lora_grad_a_kernel(AdapterArgs p) {
  GEMM_RING
  const int id = xcd_logical(blockIdx.x, p.n_tiles * p.msplit);
  const int s = id / p.n_tiles, kt = id - s * p.n_tiles;
  const int k0 = kt * TN, kb = s * p.kper, ke = min(p.rows, kb + p.kper);
  f32x16 acc[4][NI];
  gemm_tile<E, false, true>(acc, p.uT + kb, p.ld_rt, p.rank, p.big + (int64_t)kb * p.ld_big + k0, p.ld_big,
                         p.width - k0, ke - kb, s0, s1, s2, s3);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  float* part = p.part + (int64_t)s * p.rank * p.width;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int k = k0 + b_row(ni, lane, wn);
    if (k >= p.width) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = a_row(mi, i, lane, wm);
        if (r < p.rank) part[(int64_t)r * p.width + k] = acc[mi][ni][i];
      }
  }
}

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void lora_grad_b_kernel(AdapterArgs p) {
  GEMM_RING
  const int id = xcd_logical(blockIdx.x, p.n_tiles * p.msplit);
  const int s = id / p.n_tiles, nt = id - s * p.n_tiles;
  const int n0 = nt * TM, kb = s * p.kper, ke = min(p.rows, kb + p.kper);
  f32x16 acc[4][NI];
  gemm_tile<E, true, false>(acc, p.big + (int64_t)kb * p.ld_big + n0, p.ld_big, p.width - n0, p.uT + kb, p.ld_rt,
                         p.rank, ke - kb, s0, s1, s2, s3);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  float* part = p.part + (int64_t)s * p.width * p.rank;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int r = b_row(ni, lane, wn);
    if (r >= p.rank) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int n = n0 + a_row(mi, i, lane, wm);
        if (n < p.width) part[(int64_t)n * p.rank + r] = acc[mi][ni][i];
      }
  }
}

// out[e] = scale * sum_s part[s][e], splits added in order
__global__ __launch_bounds__(kThreads) void lora_reduce_kernel(const float* __restrict__ part, int msplit,
                                                               int64_t n, float scale, float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  float acc = part[e];
  for (int s = 1; s < msplit; ++s) acc += part[(int64_t)s * n + e];
  out[e] = acc * scale;
}

__global__ __launch_bounds__(kThreads) void lora_zero_kernel(float* __restrict__ out, int64_t n) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e < n) out[e] = 0.f;
}

// row ranges of the contraction for the adapter products: enough splits that
// the tiles fill the device, each range a whole number of stages and at least
// 2048 rows
inline void adapter_split(int64_t rows, int64_t tiles, int& msplit, int& kper) {
  int64_t k = (256 + tiles - 1) / tiles;
  k = std::min<int64_t>(k, std::max<int64_t>(1, rows / 2048));
  k = std::max<int64_t>(1, std::min<int64_t>(k, 64));
  int64_t per = (rows + k - 1) / k;
  per = (per + TK - 1) / TK * TK;
  msplit = (int)((rows + per - 1) / per);
  kper = (int)per;
}

inline int64_t round8(int64_t v) { return (v + 7) / 8 * 8; }
inline int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }
bool ok16(const void* p) { return ((uintptr_t)p & 15) == 0; }

struct BwdLayout {
  int64_t ld_rt, rank_bytes, part_a, part_b, dx;
  int msplit_a, kper_a, msplit_b, kper_b;
};

inline BwdLayout bwd_layout(int64_t rows, int64_t in, int64_t out, int64_t rank) {
  BwdLayout L;
  L.ld_rt = round8(rows);
  L.rank_bytes = align256(rank * L.ld_rt * 2);
  adapter_split(rows, (in + TN - 1) / TN, L.msplit_a, L.kper_a);
  adapter_split(rows, (out + TM - 1) / TM, L.msplit_b, L.kper_b);
  L.part_a = align256((int64_t)L.msplit_a * rank * in * 4);
  L.part_b = align256((int64_t)L.msplit_b * out * rank * 4);
  L.dx = align256(ts_logprob_grad_hidden_workspace(rows, in, out));
  return L;
}

}  // namespace lora
}  // namespace ts

extern "C" {

int ts_lora_fwd(const void* x, int64_t ld_x, const void* weight, int64_t ld_weight, int64_t rows,
                int64_t in_features, int64_t out_features, void* y, int64_t ld_y, int dtype, void* stream) {
  using namespace ts::lora;
  using ts::bf16;
  TS_CHECK_ARG(dtype == ts::kBF16 || dtype == ts::kF16, "ts_lora_fwd: dtype %d (bf16 or fp16)", dtype);
  TS_CHECK_ARG(rows >= 0 && in_features > 0 && out_features > 0 && rows < (1 << 30) &&
                   in_features < (1 << 20) && out_features < (1 << 24),
               "ts_lora_fwd: bad shape rows=%lld in=%lld out=%lld", (long long)rows, (long long)in_features,
               (long long)out_features);
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(x && weight && y, "ts_lora_fwd: null pointer");
  TS_CHECK_ARG(in_features % 8 == 0 && out_features % 8 == 0 && ld_x % 8 == 0 && ld_weight % 8 == 0 &&
                   ld_y % 8 == 0 && ld_x >= in_features && ld_weight >= in_features && ld_y >= out_features &&
                   ok16(x) && ok16(weight) && ok16(y),
               "ts_lora_fwd: rows must be 16-byte aligned, features and leading dimensions multiples of 8");
  TS_CHECK_ARG(255 * ld_x < (1ll << 30) && 255 * ld_weight < (1ll << 30),
               "ts_lora_fwd: leading dimensions too large for 32-bit tile offsets");
  FwdArgs p{static_cast<const bf16*>(x), ld_x, static_cast<const bf16*>(weight), ld_weight, (int)rows,
            (int)in_features, (int)out_features, (int)((rows + TN - 1) / TN),
            (int)((out_features + TM - 1) / TM), static_cast<bf16*>(y), ld_y};
  hipStream_t s = static_cast<hipStream_t>(stream);
  {
    ts::TimedLaunch timed_("lora.fwd_kernel", s);
    TS_LAUNCH_E(dtype, lora_fwd_kernel, dim3((unsigned)(p.n_mtiles * p.n_ntiles)), dim3(kGemmThreads), 0, s, p);
  }
  return ts::check_launch("ts_lora_fwd");
}

int64_t ts_lora_bwd_workspace(int64_t rows, int64_t in_features, int64_t out_features, int64_t rank) {
  if (rows <= 0 || in_features <= 0 || out_features <= 0 || rank <= 0) return 0;
  const ts::lora::BwdLayout L = ts::lora::bwd_layout(rows, in_features, out_features, rank);
  return 2 * L.rank_bytes + L.part_a + L.part_b + L.dx;
}

int ts_lora_bwd(const void* grad_out, int64_t ld_grad_out, const void* x, int64_t ld_x, const void* weight,
                int64_t ld_weight, const void* lora_a, const void* lora_b_t, int64_t rank, float scaling,
                int64_t rows, int64_t in_features, int64_t out_features, void* grad_x, int64_t ld_grad_x,
                float* grad_a, float* grad_b, void* workspace, int64_t workspace_bytes, int dtype,
                void* stream) {
  using namespace ts::lora;
  using ts::bf16;
  TS_CHECK_ARG(dtype == ts::kBF16 || dtype == ts::kF16, "ts_lora_bwd: dtype %d (bf16 or fp16)", dtype);
  TS_CHECK_ARG(rows >= 0 && in_features > 0 && out_features > 0 && rank > 0 && rank <= TN &&
                   rows < (1 << 30) && in_features < (1 << 20) && out_features < (1 << 20),
               "ts_lora_bwd: bad shape rows=%lld in=%lld out=%lld rank=%lld (rank at most %d)", (long long)rows,
               (long long)in_features, (long long)out_features, (long long)rank, TN);
  const bool want_a = grad_a != nullptr, want_b = grad_b != nullptr;
  if (rows == 0) {  // no rows: zero adapter gradients (a fill kernel, so the call stays graph-capturable)
    hipStream_t s = static_cast<hipStream_t>(stream);
    for (float* g : {want_a ? grad_a : nullptr, want_b ? grad_b : nullptr}) {
      if (!g) continue;
      const int64_t n = rank * (g == grad_a ? in_features : out_features);
      hipLaunchKernelGGL(lora_zero_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0, s,
                         g, n);
    }
    return ts::check_launch("ts_lora_bwd (no rows)");
  }
  TS_CHECK_ARG(grad_out && x, "ts_lora_bwd: null grad_out or x");
  TS_CHECK_ARG(!grad_x || weight, "ts_lora_bwd: grad_x needs the weight");
  TS_CHECK_ARG(!want_a || lora_b_t, "ts_lora_bwd: grad_a needs lora_b_t");
  TS_CHECK_ARG(!want_b || lora_a, "ts_lora_bwd: grad_b needs lora_a");
  TS_CHECK_ARG(in_features % 8 == 0 && out_features % 8 == 0 && ld_grad_out % 8 == 0 && ld_x % 8 == 0 &&
                   ld_grad_out >= out_features && ld_x >= in_features && ok16(grad_out) && ok16(x) &&
                   (!lora_a || ok16(lora_a)) && (!lora_b_t || ok16(lora_b_t)),
               "ts_lora_bwd: rows must be 16-byte aligned, features and leading dimensions multiples of 8");
  TS_CHECK_ARG(255 * ld_grad_out < (1ll << 30) && 255 * ld_x < (1ll << 30) && 255 * ts::lora::round8(rows) < (1ll << 30),
               "ts_lora_bwd: leading dimensions too large for 32-bit tile offsets");
  const BwdLayout L = bwd_layout(rows, in_features, out_features, rank);
  TS_CHECK_ARG(workspace && workspace_bytes >= ts_lora_bwd_workspace(rows, in_features, out_features, rank) &&
                   ok16(workspace),
               "ts_lora_bwd: workspace of %lld bytes, need %lld (16-byte aligned)", (long long)workspace_bytes,
               (long long)ts_lora_bwd_workspace(rows, in_features, out_features, rank));
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  bf16* uT = reinterpret_cast<bf16*>(ws);
  bf16* tT = reinterpret_cast<bf16*>(ws + L.rank_bytes);
  float* part_a = reinterpret_cast<float*>(ws + 2 * L.rank_bytes);
  float* part_b = reinterpret_cast<float*>(ws + 2 * L.rank_bytes + L.part_a);
  void* dx_ws = ws + 2 * L.rank_bytes + L.part_a + L.part_b;
  if (grad_x) {
    const int st = ts::grad_hidden_launch(grad_out, ld_grad_out, weight, ld_weight, rows, in_features, out_features,
                                          grad_x, ld_grad_x, dx_ws, L.dx, dtype, stream, "lora.grad_x_kernel",
                                          "lora.grad_x_reduce_kernel");
    if (st != TS_OK) return st;
  }
  if (!want_a && !want_b) return TS_OK;
  // u^T = (g B)^T for grad_a, t^T = (x A^T)^T for grad_b
  RankArgs rk{};
  rk.rows = (int)rows;
  rk.rank = (int)rank;
  rk.n_mtiles = (int)((rows + TM - 1) / TM);
  rk.ld_out = L.ld_rt;
  if (want_a) rk.job[rk.n_jobs++] = RankJob{static_cast<const bf16*>(grad_out), ld_grad_out,
                                            static_cast<const bf16*>(lora_b_t), out_features, (int)out_features, uT};
  if (want_b) rk.job[rk.n_jobs++] = RankJob{static_cast<const bf16*>(x), ld_x, static_cast<const bf16*>(lora_a),
                                            in_features, (int)in_features, tT};
  {
    ts::TimedLaunch timed_("lora.rank_kernel", s);
    TS_LAUNCH_E(dtype, lora_rank_kernel, dim3((unsigned)(rk.n_mtiles * rk.n_jobs)), dim3(kGemmThreads), 0, s, rk);
  }
  int st = ts::check_launch("ts_lora_bwd rank");
  if (st != TS_OK) return st;
  if (want_a) {
    AdapterArgs a{uT, L.ld_rt, static_cast<const bf16*>(x), ld_x, (int)rows, (int)rank, (int)in_features,
                  (int)((in_features + TN - 1) / TN), L.msplit_a, L.kper_a, part_a};
    {
      ts::TimedLaunch timed_("lora.grad_a_kernel", s);
      TS_LAUNCH_E(dtype, lora_grad_a_kernel, dim3((unsigned)(a.n_tiles * a.msplit)), dim3(kGemmThreads), 0, s, a);
    }
    const int64_t n = rank * in_features;
    {
      ts::TimedLaunch timed_("lora.reduce_kernel", s);
      hipLaunchKernelGGL(lora_reduce_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                         s, part_a, L.msplit_a, n, scaling, grad_a);
    }
    st = ts::check_launch("ts_lora_bwd grad_a");
    if (st != TS_OK) return st;
  }
  if (want_b) {
    AdapterArgs b{tT, L.ld_rt, static_cast<const bf16*>(grad_out), ld_grad_out, (int)rows, (int)rank,
                  (int)out_features, (int)((out_features + TM - 1) / TM), L.msplit_b, L.kper_b, part_b};
    {
      ts::TimedLaunch timed_("lora.grad_b_kernel", s);
      TS_LAUNCH_E(dtype, lora_grad_b_kernel, dim3((unsigned)(b.n_tiles * b.msplit)), dim3(kGemmThreads), 0, s, b);
    }
    const int64_t n = out_features * rank;
    {
      ts::TimedLaunch timed_("lora.reduce_kernel", s);
      hipLaunchKernelGGL(lora_reduce_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                         s, part_b, L.msplit_b, n, scaling, grad_b);
    }
    st = ts::check_launch("ts_lora_bwd grad_b");
    if (st != TS_OK) return st;
  }
  return TS_OK;
}

}  // extern "C"
