// Chunked-vocab fused log-probability / entropy and its gradient with respect
// to the hidden states, for gfx950 (bf16 operands, fp32 accumulation).
//
// Reference: accel/fused_logprob.py:61-338.  The reference materialises one
// fp32 [chunk, V] logit block per chunk and makes several passes over it; here
// the logits never leave the MFMA accumulators:
//
//   forward   logits^T tile = W_tile . H_tile^T on MFMA (A = vocab rows of W,
//             B = token rows of H, both K-contiguous).  The epilogue reduces
//             each token column of the tile to (max, sum exp, sum exp*(l-max))
//             and picks the target logit; a combine kernel merges the per-tile
//             partials into logprob, entropy and lse.  HBM traffic: W once,
//             H once per vocab super-tile, partials (12 bytes/token/tile).
//   backward  the same tile GEMM recomputes the logits; the epilogue forms
//             dlogits = -p (g_lp + g_H (log p + H)) + g_lp [v == t] in
//             registers, rounds it to bf16 (the reference rounds dlogits to the
//             hidden dtype before its VJP GEMM, fused_logprob.py:165, :295) and
//             stores a [rows, V] bf16 block; a second GEMM multiplies it by
//             W (given as W^T so both operands are K-contiguous) into dh.
//
// GEMM core (gemm_core.h): 256 x 256 work-group tiles on
// v_mfma_f32_32x32x16_bf16, K streamed through a 4-stage LDS ring by
// buffer_load ... lds.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "gemm_core.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace lp {

using namespace ts::gemm;

constexpr int kThreads = 256;      // combine / transpose kernels
constexpr int BM = TM;   // vocab rows per forward partial
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }

// (max, sum exp(l - max), sum exp(l - max) (l - max)) of two disjoint sets of
// logits, either of which may be empty (max = -inf)
__device__ __forceinline__ void merge_stats(float& m, float& s, float& e, float mo, float so, float eo) {
  if (mo == neg_inf()) return;
  if (m == neg_inf()) {
    m = mo;
    s = so;
    e = eo;
    return;
  }
  const float mn = fmaxf(m, mo);
  const float a = fast_exp2((m - mn) * kLog2e);
  const float b = fast_exp2((mo - mn) * kLog2e);
  e = a * (e + s * (m - mn)) + b * (eo + so * (mo - mn));
  s = a * s + b * so;
  m = mn;
}

// ---------------------------------------------------------------------------
// forward: per (vocab tile, token tile) partial softmax statistics
// ---------------------------------------------------------------------------
struct FwdArgs {
  const bf16* h;
  int64_t ldh;
  const bf16* w;
  int64_t ldw;
  const int64_t* target;
  int rows, dim, vocab;
  int n_ttiles, n_vtiles;
  float* part_m;   // [n_vtiles][rows]
  float* part_s;
  float* part_e;
  float* tgt;      // [rows] target logit
};

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void fwd_stats_kernel(FwdArgs p) {
  GEMM_RING
  const int total = p.n_ttiles * p.n_vtiles;
  int vt, tt;
  grouped_tile(xcd_logical(blockIdx.x, total), p.n_vtiles, p.n_ttiles, vt, tt);
  const int v0 = vt * TM, n0 = tt * TN;
  f32x16 acc[4][NI];
  gemm_tile<E, false, false>(acc, p.w + (int64_t)v0 * p.ldw, p.ldw, min(TM, p.vocab - v0),
                          p.h + (int64_t)n0 * p.ldh, p.ldh, min(TN, p.rows - n0), p.dim, s0, s1, s2, s3);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  float* xm = reinterpret_cast<float*>(s0);  // [TN] per token, from the wm = 1 waves
  float* xs = xm + TN;
  float* xe = xs + TN;
  // rows past the vocabulary (last vocab tile only) take no part
  if (v0 + TM > p.vocab) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (v0 + a_row(mi, i, lane, wm) >= p.vocab) acc[mi][ni][i] = neg_inf();
  }
  float mk[NI], sk[NI], ek[NI];  // this lane's column statistics, kept across the exchange
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = b_row(ni, lane, wn);
    float m = neg_inf();
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; i += 2) m = fmaxf(m, fmaxf(acc[mi][ni][i], acc[mi][ni][i + 1]));
    // sum of q = 2^d2 and of q d2 with d2 = (l - m) log2 e as one FMA per logit; the second
    // sum is taken back to natural-log units once
    float sum = 0.f, e = 0.f;
    const float m2 = m * kLog2e;
    if (v0 + TM <= p.vocab) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float d2 = fmaf(acc[mi][ni][i], kLog2e, -m2);
          const float q = fast_exp2(d2);
          sum += q;
          e = fmaf(q, d2, e);
        }
    } else if (m != neg_inf()) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float d2 = fmaf(acc[mi][ni][i], kLog2e, -m2);  // -inf past the vocabulary: q = 0
          const float q = fast_exp2(d2);
          sum += q;
          e = q > 0.f ? fmaf(q, d2, e) : e;
        }
    }
    e *= kLn2;
    // merge with the other half-wave (lane ^ 32 holds the other vocab rows)
    {
      const float mo = shfl_xor(m, 32), so = shfl_xor(sum, 32), eo = shfl_xor(e, 32);
      merge_stats(m, sum, e, mo, so, eo);
    }
    if (wm == 1 && lane < 32) {
      xm[col] = m;
      xs[col] = sum;
      xe[col] = e;
    }
    mk[ni] = m;
    sk[ni] = sum;
    ek[ni] = e;
  }
  __syncthreads();  // one exchange for both column groups (their columns differ)
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = b_row(ni, lane, wn);
    const int n = n0 + col;
    if (wm == 0 && lane < 32 && n < p.rows) {
      merge_stats(mk[ni], sk[ni], ek[ni], xm[col], xs[col], xe[col]);
      const int64_t o = (int64_t)vt * p.rows + n;
      p.part_m[o] = mk[ni];
      p.part_s[o] = sk[ni];
      p.part_e[o] = ek[ni];
    }
  }
}

// target logit l[n, t] = sum_d h[n, d] W[t, d] (fp32 sum of exact bf16
// products), one wave per row; rows with t outside [0, vocab) are skipped
// (the combine kernel writes NaN for them)
template <typename E>
__global__ __launch_bounds__(kThreads) void target_logit_kernel(const bf16* __restrict__ h, int64_t ldh,
                                                                const bf16* __restrict__ w, int64_t ldw,
                                                                const int64_t* __restrict__ target, int rows,
                                                                int dim, int vocab, float* __restrict__ tgt) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (n >= rows) return;
  const int64_t t = target[n];
  if (t < 0 || t >= vocab) return;
  const bf16* hr = h + (int64_t)n * ldh;
  const bf16* wr = w + t * ldw;
  float acc = 0.f;
  for (int d = 8 * lane; d < dim; d += 512) {
    const u32x4 a = ld16(hr + d), b = ld16(wr + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = fmaf(bits_to_f<E>(a[i] & 0xffffu), bits_to_f<E>(b[i] & 0xffffu), acc);
      acc = fmaf(bits_to_f<E>(a[i] >> 16), bits_to_f<E>(b[i] >> 16), acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) tgt[n] = acc;
}

// merge the per-vocab-tile partials of each token: a work-group owns 64 tokens;
// its 4 waves merge the tiles t = wave, wave + 4, ... (lanes read 64
// consecutive tokens of one tile: coalesced), then wave 0 merges the four
// partial states in wave order
__global__ __launch_bounds__(kThreads) void combine_kernel(const float* __restrict__ pm,
                                                           const float* __restrict__ ps,
                                                           const float* __restrict__ pe,
                                                           const float* __restrict__ tgt,
                                                           const int64_t* __restrict__ target,
                                                           int rows, int n_vtiles, int vocab,
                                                           float* __restrict__ logprob,
                                                           float* __restrict__ entropy,
                                                           float* __restrict__ lse) {
  __shared__ float sm[4][64], ss[4][64], se[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + lane;
  float M = neg_inf(), S = 0.f, E = 0.f;  // E: sum exp(l - M) (l - M)
  if (n < rows) {
    for (int t = wave; t < n_vtiles; t += 4) {
      const int64_t o = (int64_t)t * rows + n;
      merge_stats(M, S, E, pm[o], ps[o], pe[o]);
    }
  }
  sm[wave][lane] = M;
  ss[wave][lane] = S;
  se[wave][lane] = E;
  __syncthreads();
  if (wave != 0 || n >= rows) return;
#pragma unroll
  for (int w = 1; w < 4; ++w) merge_stats(M, S, E, sm[w][lane], ss[w][lane], se[w][lane]);
  const float logs = logf(S);
  const int64_t tg = target[n];
  const bool ok = tg >= 0 && tg < vocab;
  logprob[n] = ok ? (tgt[n] - M) - logs : __builtin_nanf("");
  lse[n] = M + logs;
  if (entropy) entropy[n] = logs - E / S;
}

// ---------------------------------------------------------------------------
// backward 1: recompute logits, form bf16 dlogits [rows, ld] (pad columns 0)
// ---------------------------------------------------------------------------
struct DlArgs {
  const bf16* h;
  int64_t ldh;
  const bf16* w;
  int64_t ldw;
  const int64_t* target;
  const float* lse;
  const float* ent;
  const float* g_lp;
  const float* g_ent;  // may be null
  int rows, dim, vocab, vocab_pad;
  int n_ttiles, n_vtiles;
  bf16* dl;
  int64_t ldl;
};

constexpr int OPITCH = TM + 8;  // staging pitch (bf16) of [64 tokens][TM vocab] quarter tiles
static_assert(64 * OPITCH <= kRingElems, "a quarter of the dlogits tile fits one ring stage");

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void dlogits_kernel(DlArgs p) {
  GEMM_RING
  const int total = p.n_ttiles * p.n_vtiles;
  int vt, tt;
  grouped_tile(xcd_logical(blockIdx.x, total), p.n_vtiles, p.n_ttiles, vt, tt);
  const int v0 = vt * TM, n0 = tt * TN;
  f32x16 acc[4][NI];
  gemm_tile<E, false, false>(acc, p.w + (int64_t)v0 * p.ldw, p.ldw, min(TM, p.vocab - v0),
                          p.h + (int64_t)n0 * p.ldh, p.ldh, min(TN, p.rows - n0), p.dim, s0, s1, s2, s3);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  // tokens 64 q .. 64 q + 63 of the tile are staged in ring stage q as [64][OPITCH]
  auto quarter = [&](int q) -> bf16* { return q == 0 ? s0 : q == 1 ? s1 : q == 2 ? s2 : s3; };
  // dl = -p (g_lp + g_H (log p + H)) + g_lp [v = t], with log2 p = l log2 e - lse log2 e as one
  // FMA and the bracket as one FMA in log2 p: A = g_H ln 2, B = g_lp + g_H H per token.  Tiles
  // inside the vocabulary and the row range (all but the last of each) skip the bounds tests.
  auto epilogue = [&](auto full_c) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = b_row(ni, lane, wn);  // token within the tile
      bf16* out = quarter(col >> 6) + (col & 63) * OPITCH;
      const int n = n0 + col;
      float lse2 = 0.f, coef_a = 0.f, coef_b = 0.f, glp = 0.f;
      int t = -1;
      if (FULL || n < p.rows) {
        lse2 = p.lse[n] * kLog2e;
        glp = p.g_lp[n];
        coef_b = glp;
        if (p.g_ent) {
          const float gent = p.g_ent[n];
          coef_a = gent * kLn2;
          coef_b = fmaf(gent, p.ent[n], glp);
        }
        const int64_t tt = p.target[n];
        t = (tt >= 0 && tt < p.vocab) ? (int)tt : -1;  // out-of-range targets match no row
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          uint32_t packed[2];
#pragma unroll
          for (int j = 0; j < 4; j += 2) {
            float d2[2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
              const int i = 4 * i4 + j + jj;
              const int v = v0 + a_row(mi, i, lane, wm);
              const float logp2 = fmaf(acc[mi][ni][i], kLog2e, -lse2);
              float d = -fast_exp2(logp2) * fmaf(coef_a, logp2, coef_b);
              if (v == t) d += glp;
              if (!FULL && !(v < p.vocab && n < p.rows)) d = 0.f;
              d2[jj] = d;
            }
            packed[j >> 1] = pack2<E>(d2[0], d2[1]);
          }
          // vocab rows a_row(mi, 4 i4 .. 4 i4 + 3) are consecutive: one 8-byte write
          *reinterpret_cast<u32x2*>(out + a_row(mi, 4 * i4, lane, wm)) = u32x2{packed[0], packed[1]};
        }
    }
  };
  if (v0 + TM <= p.vocab && n0 + TN <= p.rows) epilogue(std::true_type{});
  else epilogue(std::false_type{});
  __syncthreads();
  // coalesced store of the [TN tokens][TM vocab] tile
  const int vmax = min(TM, p.vocab_pad - v0);
#pragma unroll 4
  for (int it = 0; it < (TN * TM / 8) / kGemmThreads; ++it) {
    const int c = it * kGemmThreads + tid;
    const int row = c / (TM / 8), chunk = (c % (TM / 8)) * 8;
    const int n = n0 + row;
    if (n < p.rows && chunk < vmax)
      *reinterpret_cast<u32x4*>(p.dl + (int64_t)n * p.ldl + v0 + chunk) =
          *reinterpret_cast<const u32x4*>(quarter(row >> 6) + (row & 63) * OPITCH + chunk);
  }
}

// ---------------------------------------------------------------------------
// backward 2: grad_hidden[n][d] = sum_v dl[n][v] W[v][d] as C^T = W^T . dl^T,
// W read in place as a K-strided operand (its rows are the contraction
// index).  With `ksplit` > 1 the vocabulary is cut into ksplit ranges of
// whole stages; range s of every tile writes fp32 partial sums to
// part[s][n][d] and grad_hidden_reduce_kernel adds them in range order.
// ---------------------------------------------------------------------------
struct DhArgs {
  const bf16* w;    // [vocab][ldw]
  int64_t ldw;
  const bf16* dl;   // [rows][ldl]
  int64_t ldl;
  int rows, dim, vocab;
  int n_ttiles, n_dtiles, ksplit, kper;  // kper: vocabulary per range (multiple of TK)
  bf16* dh;
  int64_t ldd;
  float* part;      // [ksplit][rows][dim] when ksplit > 1
};

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void grad_hidden_kernel(DhArgs p) {
  GEMM_RING
  const int tiles = p.n_ttiles * p.n_dtiles;
  const int total = tiles * p.ksplit;
  const int id = xcd_logical(blockIdx.x, total);
  const int ks = id / tiles;  // vocabulary range: tiles of one range run together
  int dt, tt;
  grouped_tile(id - ks * tiles, p.n_dtiles, p.n_ttiles, dt, tt);
  const int d0 = dt * TM, n0 = tt * TN;
  const int kb = ks * p.kper, ke = min(p.vocab, kb + p.kper);
  f32x16 acc[4][NI];
  gemm_tile<E, true, false>(acc, p.w + (int64_t)kb * p.ldw + d0, p.ldw, p.dim - d0, p.dl + (int64_t)n0 * p.ldl + kb,
                         p.ldl, min(TN, p.rows - n0), ke - kb, s0, s1, s2, s3);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int n = n0 + b_row(ni, lane, wn);
    if (n >= p.rows) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d = d0 + a_row(mi, 4 * i4, lane, wm);
        const float a[4] = {acc[mi][ni][4 * i4], acc[mi][ni][4 * i4 + 1], acc[mi][ni][4 * i4 + 2],
                            acc[mi][ni][4 * i4 + 3]};
        if (p.ksplit > 1) {
          float* q = p.part + ((int64_t)ks * p.rows + n) * p.dim + d;
          if (d + 3 < p.dim) {
            *reinterpret_cast<f32x4*>(q) = f32x4{a[0], a[1], a[2], a[3]};
          } else {
            for (int j = 0; j < 4; ++j)
              if (d + j < p.dim) q[j] = a[j];
          }
        } else if (d + 3 < p.dim) {
          *reinterpret_cast<u32x2*>(p.dh + (int64_t)n * p.ldd + d) = u32x2{pack2<E>(a[0], a[1]), pack2<E>(a[2], a[3])};
        } else {
          for (int j = 0; j < 4; ++j)
            if (d + j < p.dim) reinterpret_cast<E*>(p.dh)[(int64_t)n * p.ldd + d + j] = from_f<E>(a[j]);
        }
      }
  }
}

// dh = bf16(sum_s part[s]) in range order; four elements per thread
template <typename E>
__global__ __launch_bounds__(kThreads) void grad_hidden_reduce_kernel(const float* __restrict__ part, int ksplit,
                                                                      int rows, int dim, bf16* __restrict__ dh,
                                                                      int64_t ldd) {
  const int64_t e = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
  const int64_t total = (int64_t)rows * dim;
  if (e >= total) return;
  const int64_t n = e / dim;
  const int d = (int)(e - n * dim);
  f32x4 s = *reinterpret_cast<const f32x4*>(part + e);
  for (int k = 1; k < ksplit; ++k) s += *reinterpret_cast<const f32x4*>(part + (int64_t)k * total + e);
  *reinterpret_cast<u32x2*>(dh + n * ldd + d) = u32x2{pack2<E>(s[0], s[1]), pack2<E>(s[2], s[3])};
}

// ---------------------------------------------------------------------------
// backward 3 (trainable head): grad_weight[v][d] += sum_n dl[n][v] h[n][d] in
// fp32, as C = dl^T . h with both operands K-strided (K = the block's rows);
// the epilogue adds the tile into the fp32 accumulator, so a call per block
// accumulates across blocks in block order.
// ---------------------------------------------------------------------------
struct DwArgs {
  const bf16* dl;   // [rows][ldl]
  int64_t ldl;
  const bf16* h;    // [rows][ldh]
  int64_t ldh;
  int rows, dim, vocab;
  int n_vtiles, n_dtiles;
  float* gw;        // [vocab][ldg]
  int64_t ldg;
};

template <typename E>
__global__ __launch_bounds__(kGemmThreads, 1) void grad_weight_kernel(DwArgs p) {
  GEMM_RING
  const int total = p.n_vtiles * p.n_dtiles;
  int vt, dt;
  grouped_tile(xcd_logical(blockIdx.x, total), p.n_vtiles, p.n_dtiles, vt, dt);
  const int v0 = vt * TM, d0 = dt * TN;
  f32x16 acc[4][NI];
  gemm_tile<E, true, true>(acc, p.dl + v0, p.ldl, p.vocab - v0, p.h + d0, p.ldh, p.dim - d0, p.rows, s0, s1, s2,
                        s3);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int d = d0 + b_row(ni, lane, wn);
    if (d >= p.dim) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = v0 + a_row(mi, i, lane, wm);
        if (v < p.vocab) p.gw[(int64_t)v * p.ldg + d] += acc[mi][ni][i];
      }
  }
}

// ksplit (vocabulary ranges) for grad_hidden: as many ranges as keep the
// launch within one round of 256 work-groups (one per CU) when the row tiles
// alone do not fill it -- a second, partial round would cost a whole range's
// time (80 tiles: three ranges of a third, not four of a quarter in two
// rounds) -- each range at least 4096 vocabulary rows
inline void grad_hidden_split(int64_t rows, int64_t dim, int64_t vocab, int& ksplit, int& kper) {
  const int64_t tiles = ((rows + TN - 1) / TN) * ((dim + TM - 1) / TM);
  int64_t k = 256 / tiles;
  k = std::min<int64_t>(k, std::max<int64_t>(1, vocab / 4096));
  k = std::max<int64_t>(1, std::min<int64_t>(k, 16));
  int64_t per = (vocab + k - 1) / k;
  per = (per + TK - 1) / TK * TK;
  ksplit = (int)((vocab + per - 1) / per);
  kper = (int)per;
}

bool ok16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace lp
}  // namespace ts

extern "C" {

int64_t ts_logprob_fwd_workspace(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  const int64_t vt = (vocab + ts::lp::BM - 1) / ts::lp::BM;
  return (3 * vt + 1) * rows * (int64_t)sizeof(float);
}

int ts_logprob_fwd(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                   const int64_t* target, int64_t rows, int64_t dim, int64_t vocab, float* logprob,
                   float* entropy, float* lse, void* workspace, int64_t workspace_bytes, int dtype,
                   void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(dtype == ts::kBF16 || dtype == ts::kF16, "ts_logprob_fwd: dtype %d (bf16 or fp16)", dtype);
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && vocab < (1 << 30) &&
                   dim < (1 << 20),
               "ts_logprob_fwd: bad shape rows=%lld dim=%lld vocab=%lld", (long long)rows,
               (long long)dim, (long long)vocab);
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(hidden && weight && target && logprob && lse, "ts_logprob_fwd: null pointer");
  TS_CHECK_ARG(dim % 8 == 0 && ld_hidden % 8 == 0 && ld_weight % 8 == 0 && ld_hidden >= dim &&
                   ld_weight >= dim && ok16(hidden) && ok16(weight),
               "ts_logprob_fwd: hidden/weight rows must be 16-byte aligned with dim %% 8 == 0");
  TS_CHECK_ARG(255 * ld_hidden < (1ll << 30) && 255 * ld_weight < (1ll << 30),
               "ts_logprob_fwd: leading dimensions too large for 32-bit tile offsets");
  TS_CHECK_ARG(workspace && workspace_bytes >= ts_logprob_fwd_workspace(rows, vocab),
               "ts_logprob_fwd: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
               (long long)ts_logprob_fwd_workspace(rows, vocab));
  FwdArgs a;
  a.h = (const ts::bf16*)hidden;
  a.ldh = ld_hidden;
  a.w = (const ts::bf16*)weight;
  a.ldw = ld_weight;
  a.target = target;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.n_ttiles = (int)((rows + TN - 1) / TN);
  a.n_vtiles = (int)((vocab + BM - 1) / BM);
  float* ws = (float*)workspace;
  a.part_m = ws;
  a.part_s = ws + (int64_t)a.n_vtiles * rows;
  a.part_e = ws + 2 * (int64_t)a.n_vtiles * rows;
  a.tgt = ws + 3 * (int64_t)a.n_vtiles * rows;
  TS_CHECK_ARG((int64_t)a.n_ttiles * a.n_vtiles < (1ll << 31), "ts_logprob_fwd: grid too large");
  hipStream_t s = (hipStream_t)stream;
  { ts::TimedLaunch timed_("logprob.fwd_stats_kernel", s); TS_LAUNCH_E(dtype, fwd_stats_kernel, dim3((unsigned)(a.n_ttiles * a.n_vtiles)), dim3(kGemmThreads),
                     0, s, a); }
  int st = ts::check_launch("ts_logprob_fwd (tiles)");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.target_logit_kernel", s); TS_LAUNCH_E(dtype, target_logit_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(kThreads),
                     0, s, a.h, a.ldh, a.w, a.ldw, target, (int)rows, (int)dim, (int)vocab, a.tgt); }
  st = ts::check_launch("ts_logprob_fwd (target logits)");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.combine_kernel", s); hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(kThreads),
                     0, s, a.part_m, a.part_s, a.part_e, a.tgt, target, (int)rows, a.n_vtiles,
                     (int)vocab, logprob, entropy, lse); }
  return ts::check_launch("ts_logprob_fwd (combine)");
}

int ts_logprob_dlogits(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                       const int64_t* target, const float* lse, const float* entropy,
                       const float* grad_lp, const float* grad_ent, int64_t rows, int64_t dim,
                       int64_t vocab, void* dlogits, int64_t ld_dlogits, int dtype, void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(dtype == ts::kBF16 || dtype == ts::kF16, "ts_logprob_dlogits: dtype %d (bf16 or fp16)", dtype);
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && vocab < (1 << 30) &&
                   dim < (1 << 20),
               "ts_logprob_dlogits: bad shape");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(hidden && weight && target && lse && grad_lp && dlogits,
               "ts_logprob_dlogits: null pointer");
  TS_CHECK_ARG(!grad_ent || entropy, "ts_logprob_dlogits: grad_ent needs the saved entropy");
  TS_CHECK_ARG(dim % 8 == 0 && ld_hidden % 8 == 0 && ld_weight % 8 == 0 && ok16(hidden) &&
                   ok16(weight) && ok16(dlogits) && ld_dlogits % 8 == 0 && ld_dlogits >= vocab,
               "ts_logprob_dlogits: alignment (16 bytes, dims %% 8) or ld_dlogits");
  TS_CHECK_ARG(255 * ld_hidden < (1ll << 30) && 255 * ld_weight < (1ll << 30),
               "ts_logprob_dlogits: leading dimensions too large for 32-bit tile offsets");
  DlArgs a;
  a.h = (const ts::bf16*)hidden;
  a.ldh = ld_hidden;
  a.w = (const ts::bf16*)weight;
  a.ldw = ld_weight;
  a.target = target;
  a.lse = lse;
  a.ent = entropy;
  a.g_lp = grad_lp;
  a.g_ent = grad_ent;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.vocab_pad = (int)((vocab + 7) / 8 * 8);
  a.n_ttiles = (int)((rows + TN - 1) / TN);
  a.n_vtiles = (int)((a.vocab_pad + BM - 1) / BM);
  a.dl = (ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  TS_CHECK_ARG(a.vocab_pad <= ld_dlogits, "ts_logprob_dlogits: ld_dlogits below padded vocab");
  { ts::TimedLaunch timed_("logprob.dlogits_kernel", (hipStream_t)stream); TS_LAUNCH_E(dtype, dlogits_kernel, dim3((unsigned)(a.n_ttiles * a.n_vtiles)), dim3(kGemmThreads),
                     0, (hipStream_t)stream, a); }
  return ts::check_launch("ts_logprob_dlogits");
}

int64_t ts_logprob_grad_hidden_workspace(int64_t rows, int64_t dim, int64_t vocab) {
  if (rows <= 0 || dim <= 0 || vocab <= 0) return 0;
  int ksplit, kper;
  ts::lp::grad_hidden_split(rows, dim, vocab, ksplit, kper);
  return ksplit > 1 ? (int64_t)ksplit * rows * dim * (int64_t)sizeof(float) : 0;
}

}  // extern "C"

namespace ts {

int grad_hidden_launch(const void* dlogits, int64_t ld_dlogits, const void* weight, int64_t ld_weight, int64_t rows,
                       int64_t dim, int64_t vocab, void* grad_hidden, int64_t ld_grad, void* workspace,
                       int64_t workspace_bytes, int dtype, void* stream, const char* label,
                       const char* reduce_label) {
  using namespace ts::lp;
  TS_CHECK_ARG(dtype == ts::kBF16 || dtype == ts::kF16, "ts_logprob_grad_hidden: dtype %d (bf16 or fp16)", dtype);
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && dim < (1 << 20) && vocab < (1 << 30),
               "ts_logprob_grad_hidden: bad shape");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(dlogits && weight && grad_hidden && ok16(dlogits) && ok16(weight) && ok16(grad_hidden) &&
                   ld_dlogits % 8 == 0 && ld_weight % 8 == 0 && ld_grad % 8 == 0 && dim % 8 == 0 &&
                   ld_dlogits >= (vocab + 7) / 8 * 8 && ld_weight >= dim && ld_grad >= dim,
               "ts_logprob_grad_hidden: alignment or leading dimensions");
  TS_CHECK_ARG(255 * ld_dlogits < (1ll << 30) && 31 * ld_weight < (1ll << 30),
               "ts_logprob_grad_hidden: leading dimensions too large for 32-bit tile offsets");
  DhArgs a;
  a.w = (const ts::bf16*)weight;
  a.ldw = ld_weight;
  a.dl = (const ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.n_ttiles = (int)((rows + TN - 1) / TN);
  a.n_dtiles = (int)((dim + TM - 1) / TM);
  grad_hidden_split(rows, dim, vocab, a.ksplit, a.kper);
  a.dh = (ts::bf16*)grad_hidden;
  a.ldd = ld_grad;
  a.part = (float*)workspace;
  if (a.ksplit > 1)
    TS_CHECK_ARG(workspace && workspace_bytes >= ts_logprob_grad_hidden_workspace(rows, dim, vocab) &&
                     ok16(workspace),
                 "ts_logprob_grad_hidden: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                 (long long)ts_logprob_grad_hidden_workspace(rows, dim, vocab));
  hipStream_t s = (hipStream_t)stream;
  {
    ts::TimedLaunch timed_(label, s);
    TS_LAUNCH_E(dtype, grad_hidden_kernel, dim3((unsigned)(a.n_ttiles * a.n_dtiles * a.ksplit)), dim3(kGemmThreads),
                       0, s, a);
  }
  int st = ts::check_launch("ts_logprob_grad_hidden");
  if (st != TS_OK || a.ksplit == 1) return st;
  const int64_t quads = rows * dim / 4;
  {
    ts::TimedLaunch timed_(reduce_label, s);
    TS_LAUNCH_E(dtype, grad_hidden_reduce_kernel, dim3((unsigned)((quads + kThreads - 1) / kThreads)), dim3(kThreads),
                       0, s, (const float*)workspace, a.ksplit, (int)rows, (int)dim, (ts::bf16*)grad_hidden, ld_grad);
  }
  return ts::check_launch("ts_logprob_grad_hidden (reduce)");
}

}  // namespace ts

extern "C" {

int ts_logprob_grad_hidden(const void* dlogits, int64_t ld_dlogits, const void* weight, int64_t ld_weight,
                           int64_t rows, int64_t dim, int64_t vocab, void* grad_hidden, int64_t ld_grad,
                           void* workspace, int64_t workspace_bytes, int dtype, void* stream) {
  return ts::grad_hidden_launch(dlogits, ld_dlogits, weight, ld_weight, rows, dim, vocab, grad_hidden, ld_grad,
                                workspace, workspace_bytes, dtype, stream, "logprob.grad_hidden_kernel",
                                "logprob.grad_hidden_reduce_kernel");
}

int ts_logprob_grad_weight(const void* dlogits, int64_t ld_dlogits, const void* hidden, int64_t ld_hidden,
                           int64_t rows, int64_t dim, int64_t vocab, float* grad_weight, int64_t ld_grad,
                           int dtype, void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(dtype == ts::kBF16 || dtype == ts::kF16, "ts_logprob_grad_weight: dtype %d (bf16 or fp16)", dtype);
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && dim < (1 << 20) && vocab < (1 << 30),
               "ts_logprob_grad_weight: bad shape");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(dlogits && hidden && grad_weight && ok16(dlogits) && ok16(hidden) && ld_dlogits % 8 == 0 &&
                   ld_hidden % 8 == 0 && dim % 8 == 0 && ld_dlogits >= vocab && ld_hidden >= dim &&
                   ld_grad >= dim,
               "ts_logprob_grad_weight: alignment or leading dimensions");
  TS_CHECK_ARG(31 * ld_dlogits < (1ll << 30) && 31 * ld_hidden < (1ll << 30),
               "ts_logprob_grad_weight: leading dimensions too large for 32-bit tile offsets");
  DwArgs a;
  a.dl = (const ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  a.h = (const ts::bf16*)hidden;
  a.ldh = ld_hidden;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.n_vtiles = (int)((vocab + TM - 1) / TM);
  a.n_dtiles = (int)((dim + TN - 1) / TN);
  a.gw = grad_weight;
  a.ldg = ld_grad;
  TS_CHECK_ARG((int64_t)a.n_vtiles * a.n_dtiles < (1ll << 31), "ts_logprob_grad_weight: grid too large");
  {
    ts::TimedLaunch timed_("logprob.grad_weight_kernel", (hipStream_t)stream);
    TS_LAUNCH_E(dtype, grad_weight_kernel, dim3((unsigned)(a.n_vtiles * a.n_dtiles)), dim3(kGemmThreads), 0,
                       (hipStream_t)stream, a);
  }
  return ts::check_launch("ts_logprob_grad_weight");
}

}  // extern "C"
