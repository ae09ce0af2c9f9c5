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
// Ranks above 64 run the rank and adapter products on that core too (the
// rank side of a tile holding `rank` valid rows of 256); ranks up to 64 run
// them on narrow 16-column MFMA tiles (lora_rank_narrow_kernel,
// lora_grad_{a,b}_narrow_kernel), which are bound by reading g and x (twice
// each over the backward) rather than by MFMA work the tile leaves idle.
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

// ---------------------------------------------------------------------------
// narrow ranks (at most kNarrowRank): the rank projections and adapter
// gradients on 16 x 16 x 32 MFMA tiles whose rank side is the rank rounded up
// to 16 (RB blocks of 16), instead of 256-wide tiles that hold `rank` valid
// rows.  These products read g and x once each and do 2 rank FLOP per
// element read: they are bound by HBM, and the narrow tiles leave the MFMA
// work at what they need and spread them over enough work-groups to keep
// loads in flight on every CU.
// ---------------------------------------------------------------------------
constexpr int kNarrowRank = 64;

// rank projections: out^T[r][m] = sum_k src[m][k] proj[r][k].  A work-group
// of 4 waves takes 64 rows (wave w rows 16 w ..) of one job over the whole of
// K (measured against 4 waves sharing the K of 16 rows, whose partial sums
// meet in LDS: 67 against 74 us on the C5 layer shape -- every work-group
// also reads all of proj, from L2, so fewer rows per work-group read more).
// A K block is 4 k-steps of 32: lane (g4, j16) loads k = k_blk + 32 s +
// 8 g4 .. + 7 of row j16 for step s (each load instruction reads 64
// contiguous bytes of each of the 16 rows); the B operands are proj rows
// 16 rb + j16 at the same k.  Rows past `rows` and chunks past K load as
// zeros, so the padding columns of out^T come out as exact zeros.
template <typename E, int RB>
__global__ __launch_bounds__(256) void lora_rank_narrow_kernel(RankArgs p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g4 = lane >> 4, j16 = lane & 15;
  const int n_mt = (p.rows + 63) / 64;
  const int jb = (int)blockIdx.x / n_mt;
  const RankJob job = p.job[jb];
  const int m0 = ((int)blockIdx.x - jb * n_mt) * 64 + 16 * wave;
  const int row = m0 + j16;
  const bool row_ok = row < p.rows;
  const bf16* src = job.src + (int64_t)(row_ok ? row : 0) * job.ld_src + 8 * g4;
  const bf16* proj[RB];
  bool r_ok[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = 16 * rb + j16;
    r_ok[rb] = r < p.rank;
    proj[rb] = job.proj + (int64_t)(r_ok[rb] ? r : 0) * job.ld_proj + 8 * g4;
  }
  f32x4 acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
#pragma unroll 2
  for (int k = 0; k < job.k; k += 128) {
    u32x4 a[4], b[RB][4];
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const bool k_ok = k + 32 * st + 8 * g4 < job.k;
      a[st] = row_ok && k_ok ? ld16(src + k + 32 * st) : zero;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) b[rb][st] = r_ok[rb] && k_ok ? ld16(proj[rb] + k + 32 * st) : zero;
    }
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb] = mma16<E>(as_bf16x8(a[st]), as_bf16x8(b[rb][st]), acc[rb]);
  }
  // acc[rb] lane (g4, j16): rows m0 + 4 g4 + i of rank 16 rb + j16
  const int m = m0 + 4 * g4;
  if (m >= p.ld_out) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    if (!r_ok[rb]) continue;
    *reinterpret_cast<u32x2*>(job.out + (int64_t)(16 * rb + j16) * p.ld_out + m) =
        u32x2{pack2<E>(acc[rb][0], acc[rb][1]), pack2<E>(acc[rb][2], acc[rb][3])};
  }
}

// adapter gradients over the row range [kb, kb + kper) of split s, for the
// 128 columns of tile t:
//   A side: part[s][r][k] = sum_m uT[r][m] x[m][k]
//   B side: part[s][k][r] = sum_m tT[r][m] g[m][k]
// The 4 waves split the range into 32-row steps (wave w steps w, w + 4, ...)
// and their partial sums are added through LDS in wave order.  In a step
// lane (g4, j16) loads rows 8 g4 .. 8 g4 + 7 at columns c0 + 8 j16 .. + 7
// (for each row the 16 lanes of a group read 256 contiguous bytes) and
// transposes the 8 x 8 block in registers, giving the B operands of 8 MFMAs,
// MFMA c taking column c0 + 8 j16 + c on lane j16; the A operands are the
// rank-side rows 16 rb + j16 at the step's rows 8 g4 .. + 7 (contiguous in
// uT / tT).
template <typename E, int RB, bool B_SIDE>
__device__ __forceinline__ void adapter_narrow(const AdapterArgs& p) {
  __shared__ f32x4 red[3][8][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g4 = lane >> 4, j16 = lane & 15;
  const int s = (int)blockIdx.x / p.n_tiles, t = (int)blockIdx.x - s * p.n_tiles;
  const int col = 128 * t + 8 * j16;
  const bool col_ok = col < p.width;
  const int kb = s * p.kper, ke = min(p.rows, kb + p.kper);
  const bf16* big = p.big + (col_ok ? col : 0);
  const bf16* small[RB];
  bool r_ok[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r = 16 * rb + j16;
    r_ok[rb] = r < p.rank;
    small[rb] = p.uT + (int64_t)(r_ok[rb] ? r : 0) * p.ld_rt;
  }
  f32x4 acc[8][RB];
#pragma unroll
  for (int c = 0; c < 8; ++c)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[c][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
#pragma unroll 2
  for (int m = kb + 32 * wave; m < ke; m += 128) {
    const int mr = m + 8 * g4;  // this lane's first row of the step
    u32x4 rows8[8], cols8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      rows8[i] = col_ok && mr + i < ke ? ld16(big + (int64_t)(mr + i) * p.ld_big) : zero;
    bf16x8 a[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      a[rb] = as_bf16x8(r_ok[rb] && mr < p.ld_rt ? ld16(small[rb] + mr) : zero);
    transpose8x8(rows8, cols8);  // cols8[c]: column col + c of rows mr .. mr + 7
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[c][rb] = mma16<E>(a[rb], as_bf16x8(cols8[c]), acc[c][rb]);
  }
  // waves 1..3 hand their sums to wave 0, one 16-rank block at a time
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    if (wave > 0) {
#pragma unroll
      for (int c = 0; c < 8; ++c) red[wave - 1][c][lane] = acc[c][rb];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int w = 0; w < 3; ++w) acc[c][rb] += red[w][c][lane];
    }
    __syncthreads();
  }
  // acc[c][rb] lane (g4, j16): ranks 16 rb + 4 g4 + i, column col + c
  if (wave > 0 || !col_ok) return;
  float* part = p.part + (int64_t)s * p.rank * p.width;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int r0 = 16 * rb + 4 * g4;
    if (r0 >= p.rank) continue;
    if constexpr (B_SIDE) {
      // part[s][k][r]: the lane's four ranks are consecutive
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        float* o = part + (int64_t)(col + c) * p.rank + r0;
        if (r0 + 3 < p.rank && (p.rank & 3) == 0) {
          *reinterpret_cast<f32x4*>(o) = acc[c][rb];
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (r0 + i < p.rank) o[i] = acc[c][rb][i];
        }
      }
    } else {
      // part[s][r][k]: the lane's eight columns are consecutive
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (r0 + i >= p.rank) continue;
        float* o = part + (int64_t)(r0 + i) * p.width + col;
        *reinterpret_cast<f32x4*>(o) = f32x4{acc[0][rb][i], acc[1][rb][i], acc[2][rb][i], acc[3][rb][i]};
        *reinterpret_cast<f32x4*>(o + 4) = f32x4{acc[4][rb][i], acc[5][rb][i], acc[6][rb][i], acc[7][rb][i]};
      }
    }
  }
}

// the two sides as kernels of their own (distinct names in profiles)
template <typename E, int RB>
__global__ __launch_bounds__(256) void lora_grad_a_narrow_kernel(AdapterArgs p) {
  adapter_narrow<E, RB, false>(p);
}
template <typename E, int RB>
__global__ __launch_bounds__(256) void lora_grad_b_narrow_kernel(AdapterArgs p) {
  adapter_narrow<E, RB, true>(p);
}

// row ranges of the contraction for the narrow adapter products: about 1024
// work-groups of 128 columns, ranges a whole number of 32-row steps and at
// least 512 rows
inline void narrow_split(int64_t rows, int64_t width, int& msplit, int& kper, int& tiles) {
  tiles = (int)((width + 127) / 128);
  int64_t k = (1024 + tiles - 1) / tiles;
  k = std::min<int64_t>(k, std::max<int64_t>(1, rows / 512));
  k = std::max<int64_t>(1, std::min<int64_t>(k, 256));
  int64_t per = (rows + k - 1) / k;
  per = (per + 31) / 32 * 32;
  msplit = (int)((rows + per - 1) / per);
  kper = (int)per;
}

// out[e] = scale * sum_s part[s][e], splits added in order
__global__ __launch_bounds__(kThreads) void lora_reduce_kernel(const float* __restrict__ part, int msplit,
                                                               int64_t n, float scale, float* __restrict__ out) {
  const int64_t e = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  float acc = part[e];
#pragma unroll 8
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
  int msplit_a, kper_a, msplit_b, kper_b, tiles_a, tiles_b;
};

inline BwdLayout bwd_layout(int64_t rows, int64_t in, int64_t out, int64_t rank) {
  BwdLayout L;
  L.ld_rt = round8(rows);
  L.rank_bytes = align256(rank * L.ld_rt * 2);
  if (rank <= kNarrowRank) {
    narrow_split(rows, in, L.msplit_a, L.kper_a, L.tiles_a);
    narrow_split(rows, out, L.msplit_b, L.kper_b, L.tiles_b);
  } else {
    adapter_split(rows, (in + TN - 1) / TN, L.msplit_a, L.kper_a);
    adapter_split(rows, (out + TM - 1) / TM, L.msplit_b, L.kper_b);
    L.tiles_a = (int)((in + TN - 1) / TN);
    L.tiles_b = (int)((out + TM - 1) / TM);
  }
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
  const int rb = (int)((rank + 15) / 16);  // 16-rank blocks of the narrow kernels
  {
    ts::TimedLaunch timed_("lora.rank_kernel", s);
    if (rank <= kNarrowRank) {
      const dim3 grid((unsigned)(((rows + 63) / 64) * rk.n_jobs));
#define TS_RANK_NARROW(RB)                                                                   \
  if (rb == RB) TS_LAUNCH_E_T(dtype, lora_rank_narrow_kernel, RB, grid, dim3(256), 0, s, rk);
      TS_RANK_NARROW(1) TS_RANK_NARROW(2) TS_RANK_NARROW(3) TS_RANK_NARROW(4)
#undef TS_RANK_NARROW
    } else {
      TS_LAUNCH_E(dtype, lora_rank_kernel, dim3((unsigned)(rk.n_mtiles * rk.n_jobs)), dim3(kGemmThreads), 0, s, rk);
    }
  }
  int st = ts::check_launch("ts_lora_bwd rank");
  if (st != TS_OK) return st;
  if (want_a) {
    AdapterArgs a{uT, L.ld_rt, static_cast<const bf16*>(x), ld_x, (int)rows, (int)rank, (int)in_features,
                  L.tiles_a, L.msplit_a, L.kper_a, part_a};
    {
      ts::TimedLaunch timed_("lora.grad_a_kernel", s);
      const dim3 grid((unsigned)(a.n_tiles * a.msplit));
      if (rank <= kNarrowRank) {
#define TS_ADAPTER_NARROW(RB)                                                                      \
  if (rb == RB) TS_LAUNCH_E_T(dtype, lora_grad_a_narrow_kernel, RB, grid, dim3(256), 0, s, a);
        TS_ADAPTER_NARROW(1) TS_ADAPTER_NARROW(2) TS_ADAPTER_NARROW(3) TS_ADAPTER_NARROW(4)
#undef TS_ADAPTER_NARROW
      } else {
        TS_LAUNCH_E(dtype, lora_grad_a_kernel, grid, dim3(kGemmThreads), 0, s, a);
      }
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
                  (int)out_features, L.tiles_b, L.msplit_b, L.kper_b, part_b};
    {
      ts::TimedLaunch timed_("lora.grad_b_kernel", s);
      const dim3 grid((unsigned)(b.n_tiles * b.msplit));
      if (rank <= kNarrowRank) {
#define TS_ADAPTER_NARROW(RB)                                                                     \
  if (rb == RB) TS_LAUNCH_E_T(dtype, lora_grad_b_narrow_kernel, RB, grid, dim3(256), 0, s, b);
        TS_ADAPTER_NARROW(1) TS_ADAPTER_NARROW(2) TS_ADAPTER_NARROW(3) TS_ADAPTER_NARROW(4)
#undef TS_ADAPTER_NARROW
      } else {
        TS_LAUNCH_E(dtype, lora_grad_b_kernel, grid, dim3(kGemmThreads), 0, s, b);
      }
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
