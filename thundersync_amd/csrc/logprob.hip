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
// GEMM core: 256 x 128 work-group tile, 4 waves of 128 x 64, K staged 64 at a
// time through double-buffered LDS (pitch 72 bf16: conflict-free 16-byte
// fragment reads), v_mfma_f32_32x32x16_bf16.
#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace lp {

constexpr int kThreads = 256;
constexpr int BM = 256;       // A rows per work-group
constexpr int BN = 128;       // B rows per work-group
constexpr int BK = 64;        // K per LDS stage
constexpr int PITCH = BK + 8; // LDS row pitch (elements)
constexpr int kStage = (BM + BN) * PITCH;  // elements per stage
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }
__device__ __forceinline__ u32x4 ld16(const bf16* p) { return *reinterpret_cast<const u32x4*>(p); }

// Work-groups are dispatched round-robin over the 8 XCDs; renumber them so each
// XCD runs a contiguous range of logical tiles (which share operand panels in
// that XCD's L2).
__device__ __forceinline__ int xcd_logical(int bid, int total) {
  const int per = total / 8, rem = total % 8;
  const int xcd = bid % 8, local = bid / 8;
  return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

struct Frag {
  u32x4 a[8];  // A tile: 256 rows x 64 k -> 2048 16-byte chunks, 8 per thread
  u32x4 b[4];  // B tile: 128 rows x 64 k -> 1024 chunks, 4 per thread
};

__device__ __forceinline__ void load_stage(Frag& f, const bf16* A, int64_t lda, int a_rows,
                                           const bf16* B, int64_t ldb, int b_rows, int k0, int K,
                                           int tid) {
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int c = it * kThreads + tid;
    const int row = c >> 3, kc = k0 + (c & 7) * 8;
    f.a[it] = (row < a_rows && kc < K) ? ld16(A + (int64_t)row * lda + kc) : u32x4{0u, 0u, 0u, 0u};
  }
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = it * kThreads + tid;
    const int row = c >> 3, kc = k0 + (c & 7) * 8;
    f.b[it] = (row < b_rows && kc < K) ? ld16(B + (int64_t)row * ldb + kc) : u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void store_stage(const Frag& f, bf16* lds, int tid) {
  bf16* sa = lds;
  bf16* sb = lds + BM * PITCH;
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int c = it * kThreads + tid;
    *reinterpret_cast<u32x4*>(sa + (c >> 3) * PITCH + (c & 7) * 8) = f.a[it];
  }
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = it * kThreads + tid;
    *reinterpret_cast<u32x4*>(sb + (c >> 3) * PITCH + (c & 7) * 8) = f.b[it];
  }
}

// acc[mi][ni]: 32x32 block (A rows 128 wm + 32 mi, B rows 64 wn + 32 ni).
// Lane l holds B row (l & 31) + 32 ni + 64 wn and A rows
// 8 (i >> 2) + 4 (l >> 5) + (i & 3) + 32 mi + 128 wm, i = 0..15.
__device__ __forceinline__ void gemm_tile(f32x16 acc[4][2], const bf16* A, int64_t lda, int a_rows,
                                          const bf16* B, int64_t ldb, int b_rows, int K, bf16* lds) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.f;
  const int nk = (K + BK - 1) / BK;
  Frag f;
  load_stage(f, A, lda, a_rows, B, ldb, b_rows, 0, K, tid);
  store_stage(f, lds, tid);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    if (more) load_stage(f, A, lda, a_rows, B, ldb, b_rows, (kt + 1) * BK, K, tid);
    const bf16* sa = lds + (kt & 1) * kStage;
    const bf16* sb = sa + BM * PITCH;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int kof = kk * 16 + 8 * (lane >> 5);
      bf16x8 af[4], bfr[2];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
        af[mi] = as_bf16x8(ld16(sa + (128 * wm + 32 * mi + (lane & 31)) * PITCH + kof));
#pragma unroll
      for (int ni = 0; ni < 2; ++ni)
        bfr[ni] = as_bf16x8(ld16(sb + (64 * wn + 32 * ni + (lane & 31)) * PITCH + kof));
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) acc[mi][ni] = mfma32(af[mi], bfr[ni], acc[mi][ni]);
    }
    if (more) store_stage(f, lds + ((kt + 1) & 1) * kStage, tid);
    __syncthreads();
  }
}

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

__device__ __forceinline__ int a_row(int mi, int i, int lane, int wm) {
  return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3) + 32 * mi + 128 * wm;
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

__global__ __launch_bounds__(kThreads, 1) void fwd_stats_kernel(FwdArgs p) {
  extern __shared__ __attribute__((aligned(16))) bf16 lds[];
  const int total = p.n_ttiles * p.n_vtiles;
  const int id = xcd_logical(blockIdx.x, total);
  const int tt = id % p.n_ttiles, vt = id / p.n_ttiles;
  const int v0 = vt * BM, n0 = tt * BN;
  f32x16 acc[4][2];
  gemm_tile(acc, p.w + (int64_t)v0 * p.ldw, p.ldw, min(BM, p.vocab - v0), p.h + (int64_t)n0 * p.ldh,
            p.ldh, min(BN, p.rows - n0), p.dim, lds);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  // LDS is free after the final barrier of gemm_tile
  float* xm = reinterpret_cast<float*>(lds);  // [BN] per token, from the wm = 1 waves
  float* xs = xm + BN;
  float* xe = xs + BN;
#pragma unroll
  for (int ni = 0; ni < 2; ++ni) {
    const int col = 64 * wn + 32 * ni + (lane & 31);
    const int n = n0 + col;
    const int64_t t = n < p.rows ? p.target[n] : -1;
    float m = neg_inf();
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = v0 + a_row(mi, i, lane, wm);
        if (v < p.vocab) {
          m = fmaxf(m, acc[mi][ni][i]);
          if (v == t) p.tgt[n] = acc[mi][ni][i];
        }
      }
    float s = 0.f, e = 0.f;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = v0 + a_row(mi, i, lane, wm);
        if (v < p.vocab) {
          const float d = acc[mi][ni][i] - m;
          const float q = fast_exp2(d * kLog2e);
          s += q;
          e = fmaf(q, d, e);
        }
      }
    // merge with the other half-wave (lane ^ 32 holds the other vocab rows)
    {
      const float mo = shfl_xor(m, 32), so = shfl_xor(s, 32), eo = shfl_xor(e, 32);
      merge_stats(m, s, e, mo, so, eo);
    }
    if (wm == 1 && lane < 32) {
      xm[col] = m;
      xs[col] = s;
      xe[col] = e;
    }
    __syncthreads();
    if (wm == 0 && lane < 32 && n < p.rows) {
      merge_stats(m, s, e, xm[col], xs[col], xe[col]);
      const int64_t o = (int64_t)vt * p.rows + n;
      p.part_m[o] = m;
      p.part_s[o] = s;
      p.part_e[o] = e;
    }
    __syncthreads();
  }
}

// merge the per-vocab-tile partials of each token
__global__ __launch_bounds__(kThreads) void combine_kernel(const float* __restrict__ pm,
                                                           const float* __restrict__ ps,
                                                           const float* __restrict__ pe,
                                                           const float* __restrict__ tgt,
                                                           const int64_t* __restrict__ target,
                                                           int rows, int n_vtiles, int vocab,
                                                           float* __restrict__ logprob,
                                                           float* __restrict__ entropy,
                                                           float* __restrict__ lse) {
  const int n = blockIdx.x * kThreads + threadIdx.x;
  if (n >= rows) return;
  float M = neg_inf();
  for (int t = 0; t < n_vtiles; ++t) M = fmaxf(M, pm[(int64_t)t * rows + n]);
  float S = 0.f, E = 0.f;
  for (int t = 0; t < n_vtiles; ++t) {
    const int64_t o = (int64_t)t * rows + n;
    const float m = pm[o];
    if (m == neg_inf()) continue;
    const float a = expf(m - M);
    S = fmaf(a, ps[o], S);
    E = fmaf(a, pe[o] + ps[o] * (m - M), E);
  }
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

constexpr int OPITCH = BM + 8;  // staging pitch (bf16) for the [BN][BM] dlogits tile

__global__ __launch_bounds__(kThreads, 1) void dlogits_kernel(DlArgs p) {
  extern __shared__ __attribute__((aligned(16))) bf16 lds[];
  const int total = p.n_ttiles * p.n_vtiles;
  const int id = xcd_logical(blockIdx.x, total);
  const int tt = id % p.n_ttiles, vt = id / p.n_ttiles;
  const int v0 = vt * BM, n0 = tt * BN;
  f32x16 acc[4][2];
  gemm_tile(acc, p.w + (int64_t)v0 * p.ldw, p.ldw, min(BM, p.vocab - v0), p.h + (int64_t)n0 * p.ldh,
            p.ldh, min(BN, p.rows - n0), p.dim, lds);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int ni = 0; ni < 2; ++ni) {
    const int col = 64 * wn + 32 * ni + (lane & 31);
    const int n = n0 + col;
    float lse_n = 0.f, h_n = 0.f, glp = 0.f, gent = 0.f;
    int64_t t = -1;
    if (n < p.rows) {
      lse_n = p.lse[n];
      glp = p.g_lp[n];
      if (p.g_ent) {
        gent = p.g_ent[n];
        h_n = p.ent[n];
      }
      t = p.target[n];
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
            float d = 0.f;
            if (v < p.vocab && n < p.rows) {
              const float logp = acc[mi][ni][i] - lse_n;
              const float pr = fast_exp2(logp * kLog2e);
              d = -pr * (glp + gent * (logp + h_n));
              if (v == t) d += glp;
            }
            d2[jj] = d;
          }
          packed[j >> 1] = pack_bf2(d2[0], d2[1]);
        }
        // vocab rows a_row(mi, 4 i4 .. 4 i4 + 3) are consecutive: one 8-byte write
        const int r = a_row(mi, 4 * i4, lane, wm);
        *reinterpret_cast<u32x2*>(lds + col * OPITCH + r) = u32x2{packed[0], packed[1]};
      }
  }
  __syncthreads();
  // coalesced store of the [BN tokens][BM vocab] tile
  const int vmax = min(BM, p.vocab_pad - v0);
#pragma unroll 4
  for (int it = 0; it < (BN * BM / 8) / kThreads; ++it) {
    const int c = it * kThreads + tid;
    const int row = c / (BM / 8), chunk = (c % (BM / 8)) * 8;
    const int n = n0 + row;
    if (n < p.rows && chunk < vmax)
      *reinterpret_cast<u32x4*>(p.dl + (int64_t)n * p.ldl + v0 + chunk) =
          *reinterpret_cast<const u32x4*>(lds + row * OPITCH + chunk);
  }
}

// ---------------------------------------------------------------------------
// backward 2: grad_hidden[n][d] = sum_v dl[n][v] W[v][d] as C^T = W^T . dl^T
// ---------------------------------------------------------------------------
struct DhArgs {
  const bf16* wt;   // [dim][ldt]
  int64_t ldt;
  const bf16* dl;   // [rows][ldl]
  int64_t ldl;
  int rows, dim, kdim;  // kdim = padded vocab
  int n_ttiles, n_dtiles;
  bf16* dh;
  int64_t ldd;
};

__global__ __launch_bounds__(kThreads, 1) void grad_hidden_kernel(DhArgs p) {
  extern __shared__ __attribute__((aligned(16))) bf16 lds[];
  const int total = p.n_ttiles * p.n_dtiles;
  const int id = xcd_logical(blockIdx.x, total);
  const int dt = id % p.n_dtiles, tt = id / p.n_dtiles;
  const int d0 = dt * BM, n0 = tt * BN;
  f32x16 acc[4][2];
  gemm_tile(acc, p.wt + (int64_t)d0 * p.ldt, p.ldt, min(BM, p.dim - d0), p.dl + (int64_t)n0 * p.ldl,
            p.ldl, min(BN, p.rows - n0), p.kdim, lds);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int ni = 0; ni < 2; ++ni) {
    const int n = n0 + 64 * wn + 32 * ni + (lane & 31);
    if (n >= p.rows) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d = d0 + a_row(mi, 4 * i4, lane, wm);
        if (d + 3 < p.dim) {
          const u32x2 v = {pack_bf2(acc[mi][ni][4 * i4], acc[mi][ni][4 * i4 + 1]),
                           pack_bf2(acc[mi][ni][4 * i4 + 2], acc[mi][ni][4 * i4 + 3])};
          *reinterpret_cast<u32x2*>(p.dh + (int64_t)n * p.ldd + d) = v;
        } else {
          for (int j = 0; j < 4; ++j)
            if (d + j < p.dim) p.dh[(int64_t)n * p.ldd + d + j] = from_f<bf16>(acc[mi][ni][4 * i4 + j]);
        }
      }
  }
}

// W [vocab][dim] -> W^T [dim][ld] with columns [vocab, ld) zero
__global__ __launch_bounds__(kThreads) void transpose_kernel(const bf16* __restrict__ w, int64_t ldw,
                                                             int vocab, int dim, bf16* __restrict__ wt,
                                                             int64_t ldt) {
  __shared__ uint16_t tile[64][65];
  const int v0 = blockIdx.x * 64, d0 = blockIdx.y * 64;
  const uint16_t* src = reinterpret_cast<const uint16_t*>(w);
  uint16_t* dst = reinterpret_cast<uint16_t*>(wt);
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int v = v0 + r, d = d0 + tx;
    tile[r][tx] = (v < vocab && d < dim) ? src[(int64_t)v * ldw + d] : (uint16_t)0;
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int d = d0 + r, v = v0 + tx;
    if (d < dim && v < ldt) dst[(int64_t)d * ldt + v] = tile[tx][r];
  }
}

constexpr size_t kGemmLds = 2 * kStage * sizeof(bf16);
static_assert((size_t)BN * OPITCH * sizeof(bf16) <= kGemmLds, "staging tile fits the GEMM LDS");

bool ok16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// kernels with more than 64 KB of dynamic LDS must say so before launch
int allow_lds(const void* fn, const char* what) {
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGemmLds) !=
      hipSuccess) {
    (void)hipGetLastError();
    set_error("%s: cannot reserve %zu bytes of LDS", what, kGemmLds);
    return TS_ERR_LAUNCH;
  }
  return TS_OK;
}

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
                   float* entropy, float* lse, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && vocab < (1 << 30) &&
                   dim < (1 << 20),
               "ts_logprob_fwd: bad shape rows=%lld dim=%lld vocab=%lld", (long long)rows,
               (long long)dim, (long long)vocab);
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(hidden && weight && target && logprob && lse, "ts_logprob_fwd: null pointer");
  TS_CHECK_ARG(dim % 8 == 0 && ld_hidden % 8 == 0 && ld_weight % 8 == 0 && ld_hidden >= dim &&
                   ld_weight >= dim && ok16(hidden) && ok16(weight),
               "ts_logprob_fwd: hidden/weight rows must be 16-byte aligned with dim %% 8 == 0");
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
  a.n_ttiles = (int)((rows + BN - 1) / BN);
  a.n_vtiles = (int)((vocab + BM - 1) / BM);
  float* ws = (float*)workspace;
  a.part_m = ws;
  a.part_s = ws + (int64_t)a.n_vtiles * rows;
  a.part_e = ws + 2 * (int64_t)a.n_vtiles * rows;
  a.tgt = ws + 3 * (int64_t)a.n_vtiles * rows;
  TS_CHECK_ARG((int64_t)a.n_ttiles * a.n_vtiles < (1ll << 31), "ts_logprob_fwd: grid too large");
  hipStream_t s = (hipStream_t)stream;
  int st = allow_lds((const void*)fwd_stats_kernel, "ts_logprob_fwd");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.fwd_stats_kernel", s); hipLaunchKernelGGL(fwd_stats_kernel, dim3((unsigned)(a.n_ttiles * a.n_vtiles)), dim3(kThreads),
                     kGemmLds, s, a); }
  st = ts::check_launch("ts_logprob_fwd (tiles)");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.combine_kernel", s); hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((rows + kThreads - 1) / kThreads)), dim3(kThreads),
                     0, s, a.part_m, a.part_s, a.part_e, a.tgt, target, (int)rows, a.n_vtiles,
                     (int)vocab, logprob, entropy, lse); }
  return ts::check_launch("ts_logprob_fwd (combine)");
}

int ts_logprob_weight_t(const void* weight, int64_t ld_weight, int64_t vocab, int64_t dim,
                        void* weight_t, int64_t ld_t, void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(weight && weight_t && vocab > 0 && dim > 0 && ld_weight >= dim && ld_t >= vocab &&
                   ld_t % 8 == 0 && vocab < (1 << 30) && dim < (1 << 20),
               "ts_logprob_weight_t: bad arguments vocab=%lld dim=%lld ld_t=%lld", (long long)vocab,
               (long long)dim, (long long)ld_t);
  const dim3 grid((unsigned)((ld_t + 63) / 64), (unsigned)((dim + 63) / 64));
  { ts::TimedLaunch timed_("logprob.transpose_kernel", (hipStream_t)stream); hipLaunchKernelGGL(transpose_kernel, grid, dim3(kThreads), 0, (hipStream_t)stream,
                     (const ts::bf16*)weight, ld_weight, (int)vocab, (int)dim, (ts::bf16*)weight_t,
                     ld_t); }
  return ts::check_launch("ts_logprob_weight_t");
}

int ts_logprob_dlogits(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                       const int64_t* target, const float* lse, const float* entropy,
                       const float* grad_lp, const float* grad_ent, int64_t rows, int64_t dim,
                       int64_t vocab, void* dlogits, int64_t ld_dlogits, void* stream) {
  using namespace ts::lp;
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
  a.n_ttiles = (int)((rows + BN - 1) / BN);
  a.n_vtiles = (int)((a.vocab_pad + BM - 1) / BM);
  a.dl = (ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  TS_CHECK_ARG(a.vocab_pad <= ld_dlogits, "ts_logprob_dlogits: ld_dlogits below padded vocab");
  int st = allow_lds((const void*)dlogits_kernel, "ts_logprob_dlogits");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.dlogits_kernel", (hipStream_t)stream); hipLaunchKernelGGL(dlogits_kernel, dim3((unsigned)(a.n_ttiles * a.n_vtiles)), dim3(kThreads),
                     kGemmLds, (hipStream_t)stream, a); }
  return ts::check_launch("ts_logprob_dlogits");
}

int ts_logprob_grad_hidden(const void* dlogits, int64_t ld_dlogits, const void* weight_t,
                           int64_t ld_t, int64_t rows, int64_t dim, int64_t vocab_padded,
                           void* grad_hidden, int64_t ld_grad, void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab_padded > 0 && vocab_padded % 8 == 0 &&
                   rows < (1 << 30) && dim < (1 << 20) && vocab_padded < (1 << 30),
               "ts_logprob_grad_hidden: bad shape");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(dlogits && weight_t && grad_hidden && ok16(dlogits) && ok16(weight_t) &&
                   ld_dlogits % 8 == 0 && ld_t % 8 == 0 && ld_dlogits >= vocab_padded &&
                   ld_t >= vocab_padded && ld_grad >= dim && ld_grad % 8 == 0 &&
                   ok16(grad_hidden),
               "ts_logprob_grad_hidden: alignment or leading dimensions");
  DhArgs a;
  a.wt = (const ts::bf16*)weight_t;
  a.ldt = ld_t;
  a.dl = (const ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.kdim = (int)vocab_padded;
  a.n_ttiles = (int)((rows + BN - 1) / BN);
  a.n_dtiles = (int)((dim + BM - 1) / BM);
  a.dh = (ts::bf16*)grad_hidden;
  a.ldd = ld_grad;
  int st = allow_lds((const void*)grad_hidden_kernel, "ts_logprob_grad_hidden");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.grad_hidden_kernel", (hipStream_t)stream); hipLaunchKernelGGL(grad_hidden_kernel, dim3((unsigned)(a.n_ttiles * a.n_dtiles)), dim3(kThreads),
                     kGemmLds, (hipStream_t)stream, a); }
  return ts::check_launch("ts_logprob_grad_hidden");
}

}  // extern "C"
