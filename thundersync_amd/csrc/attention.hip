// Forest / packed bottom-right-causal GQA attention for gfx950 (bf16, D = 128).
//
// One description (segments of query rows, runs of keys read in place, see
// include/thundersync_hip.h) drives three kernels:
//
//   fwd      query-stationary: a work-group owns a block of query rows of one
//            segment for GC query heads of one GQA group, streams the
//            segment's key runs through LDS 64 keys at a time (K and V tiles
//            shared by the GC heads), and keeps an online softmax per row.
//   dq       query-stationary like fwd, recomputing P from the saved LSE.
//   dkdv     key-stationary: a work-group owns 64 keys of one run and one KV
//            head, visits every segment that reads the run, and accumulates
//            dK/dV for all query heads of the group in registers -- no
//            atomics, fixed order, so the gradients are deterministic.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, lane layouts pinned by the
// layout probe test):
//   fwd/dq  S^T = K Q^T  (A = K rows from LDS, B = Q^T held in registers);
//           the accumulator layout gives each lane one query column, so the
//           softmax statistics of a query live in the four lanes that share
//           (lane & 15) and P^T is already in the B-operand layout of
//           O^T += V^T P^T.  V^T (and K^T for dQ) are fed from LDS rows
//           through an 8x8 register transpose.
//   dkdv    S = Q K^T, dP = dO V^T (A from LDS rows, B = K^T/V^T held in
//           registers); dV^T += dO^T P and dK^T += Q^T dS with dO^T / Q^T
//           from LDS rows through the register transpose.
// Both sides of every contraction use the same slot permutation of the
// contracted index, which is all the MFMA requires.
#include <type_traits>

#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace attn {

constexpr int D = 128;
constexpr int BK = 64;          // keys per tile (fwd / dq) and per dkdv block
constexpr int kThreads = 256;   // 4 waves
constexpr int PITCH = D + 8;    // LDS row pitch in elements (272 bytes)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }

__device__ __forceinline__ u32x4 ld16(const bf16* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(bf16* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// A 64 x 128 tile of K or V rows moved global -> registers -> LDS by 256
// threads; 16 consecutive threads read one 256-byte row.
struct Tile {
  u32x4 v[4];
};

__device__ __forceinline__ void tile_load(Tile& t, const bf16* base, int64_t row_stride, int nvalid,
                                          int tid) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = it * kThreads + tid;
    const int row = idx >> 4, chunk = idx & 15;
    if (row < nvalid)
      t.v[it] = ld16(base + (int64_t)row * row_stride + chunk * 8);
    else
      t.v[it] = u32x4{0u, 0u, 0u, 0u};
  }
}

__device__ __forceinline__ void tile_store(const Tile& t, bf16* lds, int tid) {
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int idx = it * kThreads + tid;
    st16(lds + (idx >> 4) * PITCH + (idx & 15) * 8, t.v[it]);
  }
}

// rows [0, 32) x 128 of a per-head query-row tensor -> LDS (256 threads, 2 loads each)
__device__ __forceinline__ void rows32_to_lds(bf16* lds, const bf16* base, int64_t row_stride,
                                              int nvalid, int tid) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    const int idx = it * kThreads + tid;
    const int row = idx >> 4, chunk = idx & 15;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (row < nvalid) v = ld16(base + (int64_t)row * row_stride + chunk * 8);
    st16(lds + row * PITCH + chunk * 8, v);
  }
}

// Eight LDS rows (row index given per slot j) at column c0, transposed: out[e]
// holds column c0 + e of the eight rows, slot j from row rows[j].
__device__ __forceinline__ void lds_rows_transposed(const bf16* lds, const int rows[8], int c0,
                                                    bf16x8 out[8]) {
  u32x4 in[8], tr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) in[j] = ld16(lds + rows[j] * PITCH + c0);
  transpose8x8(in, tr);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[e] = as_bf16x8(tr[e]);
}

// the row of slot j for lane group g: 4g + (j & 3) + 16 (j >> 2)
__device__ __forceinline__ void slot_rows(int g, int base, int rows[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) rows[j] = base + 4 * g + (j & 3) + 16 * (j >> 2);
}

__device__ __forceinline__ bf16x8 pack8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack_bf2(x[2 * i], x[2 * i + 1]);
  return as_bf16x8(r);
}

// Load a wave's 32 query rows x 128 as B operands of S^T = K Q^T:
// reg[qb][ks] = row (16 qb + (lane & 15)), columns 32 ks + 8 (lane >> 4) .. +7.
__device__ __forceinline__ void load_rows_b(bf16x8 reg[2][4], const bf16* base, int64_t row_stride,
                                            int nvalid, int lane) {
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = 16 * qb + (lane & 15);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (row < nvalid) v = ld16(base + (int64_t)row * row_stride + 32 * ks + 8 * (lane >> 4));
      reg[qb][ks] = as_bf16x8(v);
    }
  }
}

// S^T tile (64 keys x 32 rows) = K_lds Q^T: s[kb][qb] lane holds keys
// 16 kb + 4 (lane >> 4) + i, row 16 qb + (lane & 15).
__device__ __forceinline__ void tile_scores(f32x4 s[4][2], const bf16* sk, const bf16x8 qreg[2][4],
                                            int lane) {
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    s[kb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    s[kb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 a = as_bf16x8(ld16(sk + (16 * kb + (lane & 15)) * PITCH + 32 * ks + 8 * (lane >> 4)));
      s[kb][0] = mfma16(a, qreg[0][ks], s[kb][0]);
      s[kb][1] = mfma16(a, qreg[1][ks], s[kb][1]);
    }
  }
}

// Work-groups are dispatched round-robin over the 8 XCDs (linear id b runs on
// XCD b % 8), each with its own L2.  The grid is one-dimensional over
// (head chunk, work item) with the work items of one head chunk contiguous;
// within every full window of 64 ids, XCD c receives the 8 consecutive tasks
// 8c .. 8c + 7, so neighbours in the cost-sorted work list -- which read the
// same key or query rows -- share an L2.  A final partial window keeps the
// identity map.  Returns the work item; `y` receives the head chunk.
__device__ __forceinline__ int task_of(int n_items, int& y) {
  const int b = (int)blockIdx.x;
  const int total = (int)gridDim.x;
  const int base = b & ~63;
  int t = b;
  if (base + 64 <= total) {
    const int r = b & 63;
    t = base + ((r & 7) << 3) + (r >> 3);
  }
  y = t / n_items;
  return t - y * n_items;
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <int GC>
__global__ __launch_bounds__(kThreads, 2) void fwd_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                          ts_attn_rows O, float* __restrict__ lse,
                                                          int64_t lse_ld) {
  __shared__ __attribute__((aligned(16))) bf16 sk[BK * PITCH];
  __shared__ __attribute__((aligned(16))) bf16 sv[BK * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int yb;
  const int item = task_of(P.n_q_work, yb);
  const int seg_id = uniform_table(P.q_work)[2 * item];
  const int q0 = uniform_table(P.q_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const int chunks = group / GC;
  const int hk = yb / chunks;
  const int h = hk * group + (yb % chunks) * GC + (wave % GC);
  const ts_attn_segment seg = load_uniform(P.segs, seg_id);
  const int T = seg.q_len;
  const int off = seg.kv_len - seg.q_len;
  const int wq0 = q0 + 32 * (wave / GC);
  const int wg_last = min(q0 + P.q_block, T) - 1;
  const bool active = wq0 < T;
  const int w_last = min(wq0 + 32, T) - 1;
  const float c = P.scale * kLog2e;

  bf16x8 qreg[2][4];
  const bf16* qbase = (const bf16*)Q.ptr + (seg.q_row0 + wq0) * Q.row_stride + (int64_t)h * Q.head_stride;
  load_rows_b(qreg, qbase, Q.row_stride, active ? T - wq0 : 0, lane);

  f32x4 o[2][8];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int e = 0; e < 8; ++e) o[qb][e] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[2] = {neg_inf(), neg_inf()};
  float lsum[2] = {0.f, 0.f};

  for (int sp = 0; sp < seg.nspan; ++sp) {
    const ts_attn_ref ref = load_uniform(P.seg_spans, seg.span0 + sp);
    const ts_attn_run run = load_uniform(P.runs, ref.index);
    const bf16* kb0 = (const bf16*)run.k + (int64_t)hk * run.k_head_stride;
    const bf16* vb0 = (const bf16*)run.v + (int64_t)hk * run.v_head_stride;
    for (int kt0 = 0; kt0 < run.len; kt0 += BK) {
      if (ref.kpos + kt0 > off + wg_last) break;  // later keys are invisible to every row
      const int nvalid = min(BK, run.len - kt0);
      Tile tk, tv;
      tile_load(tk, kb0 + (int64_t)kt0 * run.k_row_stride, run.k_row_stride, nvalid, tid);
      tile_load(tv, vb0 + (int64_t)kt0 * run.v_row_stride, run.v_row_stride, nvalid, tid);
      __syncthreads();
      tile_store(tk, sk, tid);
      tile_store(tv, sv, tid);
      __syncthreads();
      if (!active || ref.kpos + kt0 > off + w_last) continue;

      f32x4 s[4][2];
      tile_scores(s, sk, qreg, lane);
      const bool need_mask = (kt0 + BK > run.len) || (ref.kpos + kt0 + BK - 1 > off + wq0);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float val = s[kb][qb][i] * c;
            if (need_mask) {
              const int key = kt0 + 16 * kb + 4 * (lane >> 4) + i;
              const int row = wq0 + 16 * qb + (lane & 15);
              if (key >= run.len || ref.kpos + key > off + row) val = neg_inf();
            }
            s[kb][qb][i] = val;
          }
      // online softmax, one query column per lane (shared by lanes l, l^16, l^32, l^48)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float mx = neg_inf();
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kb][qb][i]);
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float mnew = fmaxf(m[qb], mx);
        const float mref = (mnew == neg_inf()) ? 0.f : mnew;
        const float alpha = fast_exp2(m[qb] - mref);
        m[qb] = mnew;
        float ps = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(s[kb][qb][i] - mref);
            s[kb][qb][i] = p;
            ps += p;
          }
        lsum[qb] = lsum[qb] * alpha + ps;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[qb][e] *= alpha;
      }
      // O^T += V^T P^T, 32 keys per k-step
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        bf16x8 pk[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          float tmp[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) tmp[j] = s[2 * ss + (j >> 2)][qb][j & 3];
          pk[qb] = pack8(tmp);
        }
        int rows[8];
        slot_rows(lane >> 4, 32 * ss, rows);
        bf16x8 vt[8];
        lds_rows_transposed(sv, rows, 8 * (lane & 15), vt);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o[0][e] = mfma16(vt[e], pk[0], o[0][e]);
          o[1][e] = mfma16(vt[e], pk[1], o[1][e]);
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    float l = lsum[qb];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
    const int row = wq0 + 16 * qb + (lane & 15);
    if (row >= T) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    bf16* orow = (bf16*)O.ptr + (seg.q_row0 + row) * O.row_stride + (int64_t)h * O.head_stride +
                 32 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float tmp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tmp[e] = o[qb][e][i] * inv;
      st16(orow + 8 * i, as_u32x4(pack8(tmp)));
    }
    if ((lane >> 4) == 0)
      lse[(int64_t)h * lse_ld + seg.q_row0 + row] = l > 0.f ? (m[qb] + fast_log2(l)) * kLn2 : neg_inf();
  }
}

// ---------------------------------------------------------------------------
// backward preprocess: per (head, row) the pair (lse * log2(e), delta) with
// delta = sum_d dO * O (fp32); a row that saw no key (lse = -inf) gets +inf
// so that exp2(s * scale * log2(e) - lse2) is 0.  The two values of a row are
// adjacent so the backward kernels fetch a tile's statistics in one load.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void delta_kernel(ts_attn_rows O, ts_attn_rows dO,
                                                         const float* __restrict__ lse,
                                                         float* __restrict__ rowstats, int64_t lse_ld,
                                                         int64_t rows, int hq) {
  const int64_t pair = (int64_t)blockIdx.x * (kThreads / 16) + threadIdx.x / 16;
  const int sub = threadIdx.x & 15;
  const int64_t row = pair / hq;
  const int h = (int)(pair % hq);
  if (row >= rows) return;
  const u32x4 a = ld16((const bf16*)O.ptr + row * O.row_stride + (int64_t)h * O.head_stride + 8 * sub);
  const u32x4 b = ld16((const bf16*)dO.ptr + row * dO.row_stride + (int64_t)h * dO.head_stride + 8 * sub);
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc = fmaf(bf_bits_to_f(a[i] & 0xffffu), bf_bits_to_f(b[i] & 0xffffu), acc);
    acc = fmaf(bf_bits_to_f(a[i] >> 16), bf_bits_to_f(b[i] >> 16), acc);
  }
#pragma unroll
  for (int msk = 8; msk >= 1; msk >>= 1) acc += shfl_xor(acc, msk);
  if (sub == 0) {
    const int64_t at = (int64_t)h * lse_ld + row;
    const float l = lse[at];
    rowstats[2 * at] = l == neg_inf() ? __builtin_huge_valf() : l * kLog2e;
    rowstats[2 * at + 1] = acc;
  }
}

// ---------------------------------------------------------------------------
// backward dQ (query-stationary)
// ---------------------------------------------------------------------------
template <int GC>
__global__ __launch_bounds__(kThreads, 1) void dq_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                         ts_attn_rows dO, const float* __restrict__ rowstats,
                                                         int64_t lse_ld, ts_attn_rows dQ) {
  __shared__ __attribute__((aligned(16))) bf16 sk[BK * PITCH];
  __shared__ __attribute__((aligned(16))) bf16 sv[BK * PITCH];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int yb;
  const int item = task_of(P.n_q_work, yb);
  const int seg_id = uniform_table(P.q_work)[2 * item];
  const int q0 = uniform_table(P.q_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const int chunks = group / GC;
  const int hk = yb / chunks;
  const int h = hk * group + (yb % chunks) * GC + (wave % GC);
  const ts_attn_segment seg = load_uniform(P.segs, seg_id);
  const int T = seg.q_len;
  const int off = seg.kv_len - seg.q_len;
  const int wq0 = q0 + 32 * (wave / GC);
  const int wg_last = min(q0 + P.q_block, T) - 1;
  const bool active = wq0 < T;
  const int w_last = min(wq0 + 32, T) - 1;
  const float c = P.scale * kLog2e;

  bf16x8 qreg[2][4], dreg[2][4];
  const int64_t qoff = (seg.q_row0 + wq0);
  load_rows_b(qreg, (const bf16*)Q.ptr + qoff * Q.row_stride + (int64_t)h * Q.head_stride, Q.row_stride,
              active ? T - wq0 : 0, lane);
  load_rows_b(dreg, (const bf16*)dO.ptr + qoff * dO.row_stride + (int64_t)h * dO.head_stride,
              dO.row_stride, active ? T - wq0 : 0, lane);
  float lse2[2], dlt[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = wq0 + 16 * qb + (lane & 15);
    lse2[qb] = __builtin_huge_valf();
    dlt[qb] = 0.f;
    if (active && row < T) {
      const int64_t at = 2 * ((int64_t)h * lse_ld + seg.q_row0 + row);
      lse2[qb] = rowstats[at];
      dlt[qb] = rowstats[at + 1];
    }
  }
  f32x4 acc[2][8];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[qb][e] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int sp = 0; sp < seg.nspan; ++sp) {
    const ts_attn_ref ref = load_uniform(P.seg_spans, seg.span0 + sp);
    const ts_attn_run run = load_uniform(P.runs, ref.index);
    const bf16* kb0 = (const bf16*)run.k + (int64_t)hk * run.k_head_stride;
    const bf16* vb0 = (const bf16*)run.v + (int64_t)hk * run.v_head_stride;
    for (int kt0 = 0; kt0 < run.len; kt0 += BK) {
      if (ref.kpos + kt0 > off + wg_last) break;
      const int nvalid = min(BK, run.len - kt0);
      Tile tk, tv;
      tile_load(tk, kb0 + (int64_t)kt0 * run.k_row_stride, run.k_row_stride, nvalid, tid);
      tile_load(tv, vb0 + (int64_t)kt0 * run.v_row_stride, run.v_row_stride, nvalid, tid);
      __syncthreads();
      tile_store(tk, sk, tid);
      tile_store(tv, sv, tid);
      __syncthreads();
      if (!active || ref.kpos + kt0 > off + w_last) continue;

      f32x4 s[4][2], dp[4][2];
      tile_scores(s, sk, qreg, lane);
      tile_scores(dp, sv, dreg, lane);  // dP^T = V dO^T, same shape as S^T
      const bool need_mask = (kt0 + BK > run.len) || (ref.kpos + kt0 + BK - 1 > off + wq0);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float p = fast_exp2(s[kb][qb][i] * c - lse2[qb]);
            if (need_mask) {
              const int key = kt0 + 16 * kb + 4 * (lane >> 4) + i;
              const int row = wq0 + 16 * qb + (lane & 15);
              if (key >= run.len || ref.kpos + key > off + row) p = 0.f;
            }
            s[kb][qb][i] = p * (dp[kb][qb][i] - dlt[qb]);  // dS^T
          }
      // dQ^T += K^T dS^T, 32 keys per k-step
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        bf16x8 dsk[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          float tmp[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) tmp[j] = s[2 * ss + (j >> 2)][qb][j & 3];
          dsk[qb] = pack8(tmp);
        }
        int rows[8];
        slot_rows(lane >> 4, 32 * ss, rows);
        bf16x8 kt[8];
        lds_rows_transposed(sk, rows, 8 * (lane & 15), kt);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          acc[0][e] = mfma16(kt[e], dsk[0], acc[0][e]);
          acc[1][e] = mfma16(kt[e], dsk[1], acc[1][e]);
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = wq0 + 16 * qb + (lane & 15);
    if (row >= T) continue;
    bf16* drow = (bf16*)dQ.ptr + (seg.q_row0 + row) * dQ.row_stride + (int64_t)h * dQ.head_stride +
                 32 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float tmp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tmp[e] = acc[qb][e][i] * P.scale;
      st16(drow + 8 * i, as_u32x4(pack8(tmp)));
    }
  }
}

// ---------------------------------------------------------------------------
// backward dK / dV (key-stationary)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads, 2) void dkdv_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                           ts_attn_rows dO, const float* __restrict__ rowstats,
                                                           int64_t lse_ld) {
  __shared__ __attribute__((aligned(16))) bf16 sq[32 * PITCH];
  __shared__ __attribute__((aligned(16))) bf16 sd[32 * PITCH];
  __shared__ float s_lse2[32];
  __shared__ float s_dlt[32];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int hk;
  const int item = task_of(P.n_kv_work, hk);
  const int run_id = uniform_table(P.kv_work)[2 * item];
  const int k0 = uniform_table(P.kv_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const ts_attn_run run = load_uniform(P.runs, run_id);
  const int wk0 = k0 + 16 * wave;                 // first key (run-local) of this wave
  const int mykey = wk0 + (lane & 15);            // key column this lane holds
  const bool wave_has_keys = wk0 < run.len;
  const float c = P.scale * kLog2e;

  // K^T / V^T B operands: key (lane & 15), d = 32 ks + 8 (lane >> 4) .. +7
  bf16x8 kreg[4], vreg[4];
  {
    const bf16* kp = (const bf16*)run.k + (int64_t)mykey * run.k_row_stride + (int64_t)hk * run.k_head_stride;
    const bf16* vp = (const bf16*)run.v + (int64_t)mykey * run.v_row_stride + (int64_t)hk * run.v_head_stride;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      u32x4 a = u32x4{0u, 0u, 0u, 0u}, b = u32x4{0u, 0u, 0u, 0u};
      if (mykey < run.len) {
        a = ld16(kp + 32 * ks + 8 * (lane >> 4));
        b = ld16(vp + 32 * ks + 8 * (lane >> 4));
      }
      kreg[ks] = as_bf16x8(a);
      vreg[ks] = as_bf16x8(b);
    }
  }
  f32x4 dk[8], dv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dk[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[e] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  for (int vi = 0; vi < run.nvisit; ++vi) {
    const ts_attn_ref ref = load_uniform(P.run_visits, run.visit0 + vi);
    const ts_attn_segment seg = load_uniform(P.segs, ref.index);
    const int T = seg.q_len;
    const int off = seg.kv_len - seg.q_len;
    // row r sees key k iff kpos + k <= off + r
    int r_start = ref.kpos + k0 - off;
    if (r_start < 0) r_start = 0;
    r_start &= ~31;
    for (int r0 = r_start; r0 < T; r0 += 32) {
      const int nrows = min(32, T - r0);
      // the wave's keys are all invisible to this block when its first key
      // is beyond the block's last row
      const bool wave_active = wave_has_keys && (ref.kpos + wk0 <= off + r0 + nrows - 1);
      for (int g = 0; g < group; ++g) {
        const int h = hk * group + g;
        __syncthreads();
        const int64_t row0 = seg.q_row0 + r0;
        rows32_to_lds(sq, (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)h * Q.head_stride,
                      Q.row_stride, nrows, tid);
        rows32_to_lds(sd, (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)h * dO.head_stride,
                      dO.row_stride, nrows, tid);
        if (tid < 32) {
          float l2 = __builtin_huge_valf(), dl = 0.f;
          if (tid < nrows) {
            const int64_t at = 2 * ((int64_t)h * lse_ld + row0 + tid);
            l2 = rowstats[at];
            dl = rowstats[at + 1];
          }
          s_lse2[tid] = l2;
          s_dlt[tid] = dl;
        }
        __syncthreads();
        if (!wave_active) continue;

        // S = Q K^T and dP = dO V^T: [qb] lane holds rows 16 qb + 4 (lane >> 4) + i, key (lane & 15)
        f32x4 s[2], dp[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          s[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < 4; ++ks) {
            const int r = 16 * qb + (lane & 15);
            const bf16x8 aq = as_bf16x8(ld16(sq + r * PITCH + 32 * ks + 8 * (lane >> 4)));
            const bf16x8 ad = as_bf16x8(ld16(sd + r * PITCH + 32 * ks + 8 * (lane >> 4)));
            s[qb] = mfma16(aq, kreg[ks], s[qb]);
            dp[qb] = mfma16(ad, vreg[ks], dp[qb]);
          }
        }
        float pv[8], dsv[8];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rl = 16 * qb + 4 * (lane >> 4) + i;
            float p = fast_exp2(s[qb][i] * c - s_lse2[rl]);
            if (rl >= nrows || mykey >= run.len || ref.kpos + mykey > off + r0 + rl) p = 0.f;
            pv[4 * qb + i] = p;
            dsv[4 * qb + i] = p * (dp[qb][i] - s_dlt[rl]);
          }
        const bf16x8 pk = pack8(pv);
        const bf16x8 dsk = pack8(dsv);
        int rows[8];
        slot_rows(lane >> 4, 0, rows);
        bf16x8 at[8];
        lds_rows_transposed(sd, rows, 8 * (lane & 15), at);
#pragma unroll
        for (int e = 0; e < 8; ++e) dv[e] = mfma16(at[e], pk, dv[e]);
        lds_rows_transposed(sq, rows, 8 * (lane & 15), at);
#pragma unroll
        for (int e = 0; e < 8; ++e) dk[e] = mfma16(at[e], dsk, dk[e]);
      }
    }
  }
  if (mykey >= run.len) return;
  if (run.dk) {
    bf16* p = (bf16*)run.dk + (int64_t)mykey * run.dk_row_stride + (int64_t)hk * run.dk_head_stride +
              32 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float tmp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tmp[e] = dk[e][i] * P.scale;
      st16(p + 8 * i, as_u32x4(pack8(tmp)));
    }
  }
  if (run.dv) {
    bf16* p = (bf16*)run.dv + (int64_t)mykey * run.dv_row_stride + (int64_t)hk * run.dv_head_stride +
              32 * (lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float tmp[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) tmp[e] = dv[e][i];
      st16(p + 8 * i, as_u32x4(pack8(tmp)));
    }
  }
}

// ---------------------------------------------------------------------------
// backward dK / dV, one wave per query head (GQA groups that are a multiple of 4)
//
// A work-group owns 16 KB keys of one run and one KV head; wave w handles query
// heads w, w + 4, ... of the group over all of them, so a wave's LDS reads of
// its head's Q/dO tile feed 16 KB keys of MFMA work.  K^T operands stay in
// registers; the V tile sits in LDS.  Each wave streams its head's 32-row
// Q/dO tiles and their 32 (lse * log2 e, delta) pairs into its own
// double-buffered LDS region with buffer_load ... lds: the buffer resource of
// a tile covers exactly its valid rows, so rows past a segment's end arrive
// as zeros (no clamping, no masking: a zero row has S = dP = 0, statistics
// (0, 0), hence dS = 0 and a zero dO row, and adds nothing), and every
// lane's address is a constant byte offset fixed at kernel start.  Rows are
// 256 bytes, 16-byte chunk c of row r at chunk slot c ^ (r & 15): row reads of
// 16 rows at one chunk, transpose reads and the DMA's 4-row instructions are
// all conflict-free.  dO^T and Q^T come from ds_read_b64_tr_b16: within each
// 16-lane group, lane i receives column (i & 3) of the rows addressed by
// lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12, so lane j addressing row kbase +
// j/4, columns m0 + 4 (j & 3) yields X[kbase + t][m0 + i], t = 0..3 (pinned
// by the LDS probe test).  The causal mask is applied only to tiles that
// cross the diagonal.  The per-head partials are summed across waves through
// LDS in wave order.
// ---------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int kTile32 = 32 * D;              // elements of one 32-row tile (256-byte rows)
constexpr int kStage32 = 2 * kTile32 + 128;  // Q tile + dO tile + 32 (lse2, delta) pairs

__device__ __forceinline__ u32x2 tr_read(const bf16* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  u32x2 r;
  __builtin_memcpy(&r, &v, 8);
  return r;
}

struct Cursor {
  int vi;  // visit index; == nvisit at the end
  int r0;  // first row of the block
};

template <int KB>
__global__ __launch_bounds__(kThreads, 1) void dkdv_wave_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                                ts_attn_rows dO,
                                                                const float* __restrict__ rowstats,
                                                                int64_t lse_ld) {
  __shared__ __attribute__((aligned(16))) bf16 s_v[16 * KB * D];
  // per wave and stage: Q tile, dO tile, then 32 (lse2, delta) pairs
  __shared__ __attribute__((aligned(16))) bf16 s_b0[4][kStage32];
  __shared__ __attribute__((aligned(16))) bf16 s_b1[4][kStage32];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, j16 = lane & 15;
  int hk;
  const int item = task_of(P.n_kv_work, hk);
  const int run_id = uniform_table(P.kv_work)[2 * item];
  const int k0 = uniform_table(P.kv_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const ts_attn_run run = load_uniform(P.runs, run_id);
  constexpr int NK = 16 * KB;  // keys per work-group
  const int nkeys = min(NK, run.len - k0);
  const float c = P.scale * kLog2e;

  // per-lane LDS offsets (elements)
  int ro[4], to[8], dchunk[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ro[ks] = j16 * D + (((4 * ks + g4) ^ j16) << 3);
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int r = 4 * g4 + (j16 >> 2);
    const int col = 16 * mb + 4 * (j16 & 3);
    to[mb] = r * D + ((((col >> 3) ^ r) & 15) << 3) + (col & 7);
  }
  // DMA instruction t fills rows 4t .. 4t + 3; lane (g4, j16) the row 4t + g4,
  // chunk slot j16 with logical chunk j16 ^ (4 (t & 3) + g4)
#pragma unroll
  for (int t = 0; t < 4; ++t) dchunk[t] = (j16 ^ (4 * t + g4)) << 3;
  // byte offsets of this lane's row and chunk within a 16-row half tile
  int qoff[4], doff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    qoff[t] = (int)(((4 * t + g4) * Q.row_stride + dchunk[t]) * 2);
    doff[t] = (int)(((4 * t + g4) * dO.row_stride + dchunk[t]) * 2);
  }

  // V tile (rows past the run arrive as zeros); wave w issues instructions w, w + 4, ...
  {
    const bf16* vb = (const bf16*)run.v + (int64_t)k0 * run.v_row_stride + (int64_t)hk * run.v_head_stride;
    const rsrc_t rv = make_rsrc(vb, (uint32_t)(nkeys * run.v_row_stride * 2));
    for (int t = wave; t < 4 * KB; t += 4)
      buffer_dma16(rv, s_v + t * 512, (int)(((4 * t + g4) * run.v_row_stride + dchunk[t & 3]) * 2));
  }
  // K^T operands: kreg[kb][ks] = K[k0 + 16 kb + j16][32 ks + 8 g4 ..]
  bf16x8 kreg[KB][4];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = 16 * kb + j16;
    const bf16* kp = (const bf16*)run.k + (int64_t)(k0 + key) * run.k_row_stride + (int64_t)hk * run.k_head_stride;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
      kreg[kb][ks] = as_bf16x8(key < nkeys ? ld16(kp + 32 * ks + 8 * g4) : u32x4{0u, 0u, 0u, 0u});
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  f32x4 dk[8][KB], dv[8][KB];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      dk[mb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      dv[mb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  // first block at or after (vi, r0); skips visits with no visible rows
  auto settle = [&](Cursor cur) -> Cursor {
    while (cur.vi < run.nvisit) {
      const ts_attn_ref ref = load_uniform(P.run_visits, run.visit0 + cur.vi);
      const ts_attn_segment seg = load_uniform(P.segs, ref.index);
      if (cur.r0 < 0) {
        int rs = ref.kpos + k0 - (seg.kv_len - seg.q_len);
        rs = rs < 0 ? 0 : rs;
        cur.r0 = rs & ~31;
      }
      if (cur.r0 < seg.q_len) return cur;
      ++cur.vi;
      cur.r0 = -1;
    }
    return cur;
  };
  auto issue = [&](Cursor cur, int h, bf16* buf) {
    const ts_attn_ref ref = load_uniform(P.run_visits, run.visit0 + cur.vi);
    const ts_attn_segment seg = load_uniform(P.segs, ref.index);
    const int nrows = min(32, seg.q_len - cur.r0);
    const int n_lo = min(16, nrows), n_hi = nrows - n_lo;
    const int64_t row0 = seg.q_row0 + cur.r0;
    const bf16* qb = (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)h * Q.head_stride;
    const bf16* db = (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)h * dO.head_stride;
    const rsrc_t q_lo = make_rsrc(qb, (uint32_t)(n_lo * Q.row_stride * 2));
    const rsrc_t q_hi = make_rsrc(qb + 16 * Q.row_stride, (uint32_t)(n_hi * Q.row_stride * 2));
    const rsrc_t d_lo = make_rsrc(db, (uint32_t)(n_lo * dO.row_stride * 2));
    const rsrc_t d_hi = make_rsrc(db + 16 * dO.row_stride, (uint32_t)(n_hi * dO.row_stride * 2));
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      buffer_dma16(q_lo, buf + t * 512, qoff[t]);
      buffer_dma16(q_hi, buf + (4 + t) * 512, qoff[t]);
      buffer_dma16(d_lo, buf + kTile32 + t * 512, doff[t]);
      buffer_dma16(d_hi, buf + kTile32 + (4 + t) * 512, doff[t]);
    }
    // 32 rows x 8 bytes of statistics: lanes 0..15, 16 bytes each
    const rsrc_t rs = make_rsrc(rowstats + 2 * ((int64_t)h * lse_ld + row0), (uint32_t)(nrows * 8));
    if (lane < 16) buffer_dma16(rs, buf + 2 * kTile32, lane * 16);
  };

  // one 32-row block of the current head; buffer roles fixed per call
  auto step = [&](auto bsel, Cursor& cur, int h) {
      const ts_attn_ref ref = load_uniform(P.run_visits, run.visit0 + cur.vi);
      const ts_attn_segment seg = load_uniform(P.segs, ref.index);
      const int off = seg.kv_len - seg.q_len;
      const int r0 = cur.r0;
      Cursor nxt = settle(Cursor{cur.vi, cur.r0 + 32});
      __builtin_amdgcn_s_waitcnt(0);  // this block's tiles have landed
      // static buffer roles: the LDS reads below and the prefetch into the other
      // buffer touch different arrays, so no wait for the prefetch is needed
      bf16* cur_buf = bsel.value == 0 ? s_b0[wave] : s_b1[wave];
      bf16* nxt_buf = bsel.value == 0 ? s_b1[wave] : s_b0[wave];
      if (nxt.vi < run.nvisit) issue(nxt, h, nxt_buf);
      const bf16* tq = cur_buf;
      const bf16* td = cur_buf + kTile32;
      const float* sl = reinterpret_cast<const float*>(cur_buf + 2 * kTile32);  // [32] (lse2, delta)

      // S = Q K^T, dP = dO V^T: [qb][kb] holds rows 16 qb + 4 g4 + i, key 16 kb + j16
      f32x4 sc[2][KB], dp[2][KB];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          sc[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        bf16x8 aq[2], ad[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          aq[qb] = as_bf16x8(ld16(tq + ro[ks] + 16 * qb * D));
          ad[qb] = as_bf16x8(ld16(td + ro[ks] + 16 * qb * D));
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const bf16x8 vb = as_bf16x8(ld16(s_v + ro[ks] + 16 * kb * D));
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            sc[qb][kb] = mfma16(aq[qb], kreg[kb][ks], sc[qb][kb]);
            dp[qb][kb] = mfma16(ad[qb], vb, dp[qb][kb]);
          }
        }
      }
      // this lane's rows: 16 qb + 4 g4 + i
      float l2[2][4], dl[2][4];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rl = 16 * qb + 4 * g4 + i;
          l2[qb][i] = sl[2 * rl];
          dl[qb][i] = sl[2 * rl + 1];
        }
      // P and dS as B operands: slot j = 4 qb + i  <->  row 16 qb + 4 g4 + i
      bf16x8 pk[KB], dsk[KB];
      if (ref.kpos + k0 + NK - 1 > off + r0) {  // the block crosses the diagonal
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          const int lim = off + r0 - ref.kpos - (k0 + 16 * kb + j16);  // row rl sees the key iff rl >= -lim
          float pv[8], dsv[8];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int rl = 16 * qb + 4 * g4 + i;
              const float p = rl + lim >= 0 ? fast_exp2(sc[qb][kb][i] * c - l2[qb][i]) : 0.f;
              pv[4 * qb + i] = p;
              dsv[4 * qb + i] = p * (dp[qb][kb][i] - dl[qb][i]);
            }
          pk[kb] = pack8(pv);
          dsk[kb] = pack8(dsv);
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          float pv[8], dsv[8];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float p = fast_exp2(sc[qb][kb][i] * c - l2[qb][i]);
              pv[4 * qb + i] = p;
              dsv[4 * qb + i] = p * (dp[qb][kb][i] - dl[qb][i]);
            }
          pk[kb] = pack8(pv);
          dsk[kb] = pack8(dsv);
        }
      }
      // dV^T += dO^T P, dK^T += Q^T dS: rows d = 16 mb + 4 g4 + i, column key
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const u32x2 a0 = tr_read(td + to[mb]), a1 = tr_read(td + to[mb] + 16 * D);
        const u32x2 b0 = tr_read(tq + to[mb]), b1 = tr_read(tq + to[mb] + 16 * D);
        const bf16x8 a_do = as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
        const bf16x8 a_q = as_bf16x8(u32x4{b0[0], b0[1], b1[0], b1[1]});
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          dv[mb][kb] = mfma16(a_do, pk[kb], dv[mb][kb]);
          dk[mb][kb] = mfma16(a_q, dsk[kb], dk[mb][kb]);
        }
      }
      cur = nxt;
  };

  for (int g = wave; g < group; g += 4) {
    const int h = hk * group + g;
    Cursor cur = settle(Cursor{0, -1});
    if (cur.vi < run.nvisit) issue(cur, h, s_b0[wave]);
    while (cur.vi < run.nvisit) {
      step(std::integral_constant<int, 0>{}, cur, h);
      if (cur.vi >= run.nvisit) break;
      step(std::integral_constant<int, 1>{}, cur, h);
    }
  }

  // sum the waves' partials in wave order: wave w stages [NK keys][128 d] fp32
  // (16-byte chunk c of key k at slot c ^ (k & 31)) in s_b0[2w] (w < 2) or
  // s_b1[2(w - 2)], 2 x kStage32 bf16 >= 32 KB; every thread then adds the
  // four partials of its outputs
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  auto stage = [&](int w) -> float* {
    return reinterpret_cast<float*>(w < 2 ? s_b0[2 * w] : s_b1[2 * (w - 2)]);
  };
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    float* mine = stage(wave);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int key = 16 * kb + j16;
        const int chunk = 4 * mb + g4;  // d = 16 mb + 4 g4 .. +3
        *reinterpret_cast<f32x4*>(mine + key * D + ((chunk ^ (key & 31)) << 2)) =
            which == 0 ? dk[mb][kb] : dv[mb][kb];
      }
    __syncthreads();
    const uint64_t base = which == 0 ? run.dk : run.dv;
    const int64_t rs = which == 0 ? run.dk_row_stride : run.dv_row_stride;
    const int64_t hs = which == 0 ? run.dk_head_stride : run.dv_head_stride;
    const float mult = which == 0 ? P.scale : 1.f;
#pragma unroll
    for (int t = 0; t < KB; ++t) {
      const int e = t * kThreads + tid;  // NK x 16 outputs of 8 elements
      const int key = e >> 4, d8 = (e & 15) * 8;
      float acc8[8];
#pragma unroll
      for (int hc = 0; hc < 2; ++hc) {
        const int chunk = (d8 >> 2) + hc;
        const int slot = key * D + ((chunk ^ (key & 31)) << 2);
        f32x4 sum = *reinterpret_cast<const f32x4*>(stage(0) + slot);
#pragma unroll
        for (int w = 1; w < 4; ++w) sum += *reinterpret_cast<const f32x4*>(stage(w) + slot);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc8[4 * hc + q] = sum[q] * mult;
      }
      if (base && key < nkeys)
        st16((bf16*)base + (int64_t)(k0 + key) * rs + (int64_t)hk * hs + d8, as_u32x4(pack8(acc8)));
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
int heads_per_block(int group) {
  if (group % 4 == 0) return 4;
  if (group % 2 == 0) return 2;
  return 1;
}

// keys per dK/dV work-group: 48 for the one-wave-per-head kernel (its 192
// dK/dV accumulators and 48 S/dP values fill the 256 AGPRs), else 64
int kv_block_keys(int group) { return group % 4 == 0 ? 48 : BK; }

bool aligned_rows(const ts_attn_rows& r) {
  return r.ptr && (r.ptr % 16 == 0) && (r.row_stride % 8 == 0) && (r.head_stride % 8 == 0) &&
         r.row_stride > 0;
}

int validate(const ts_attn_problem* p, const char* what) {
  TS_CHECK_ARG(p != nullptr, "%s: null problem", what);
  TS_CHECK_ARG(p->head_dim == D, "%s: head_dim %d unsupported (128 only)", what, p->head_dim);
  TS_CHECK_ARG(p->hq > 0 && p->hkv > 0 && p->hq % p->hkv == 0, "%s: hq %d not a multiple of hkv %d",
               what, p->hq, p->hkv);
  const int gc = heads_per_block(p->hq / p->hkv);
  TS_CHECK_ARG(p->q_block == 32 * 4 / gc, "%s: q_block %d, expected %d for group %d", what,
               p->q_block, 32 * 4 / gc, p->hq / p->hkv);
  TS_CHECK_ARG(p->kv_block == kv_block_keys(p->hq / p->hkv), "%s: kv_block %d, expected %d", what,
               p->kv_block, kv_block_keys(p->hq / p->hkv));
  TS_CHECK_ARG(p->n_q_work >= 0 && p->n_kv_work >= 0 && p->n_segs >= 0 && p->n_runs >= 0,
               "%s: negative table size", what);
  TS_CHECK_ARG(p->n_q_work == 0 || (p->q_work && p->segs && p->seg_spans && p->runs),
               "%s: null table", what);
  TS_CHECK_ARG((int64_t)p->n_q_work * (p->hq / gc) < (1ll << 31) && (int64_t)p->n_kv_work * p->hkv < (1ll << 31),
               "%s: work list too long", what);
  return TS_OK;
}

}  // namespace attn
}  // namespace ts

extern "C" {

int ts_attn_heads_per_block(int group) { return group > 0 ? ts::attn::heads_per_block(group) : 0; }

int ts_attn_kv_block(int group) { return group > 0 ? ts::attn::kv_block_keys(group) : 0; }

int ts_attn_fwd(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out, float* lse,
                int64_t lse_ld, void* stream) {
  using namespace ts::attn;
  int st = validate(problem, "ts_attn_fwd");
  if (st != TS_OK) return st;
  const ts_attn_problem& P = *problem;
  if (P.n_q_work == 0) return TS_OK;
  TS_CHECK_ARG(aligned_rows(q) && aligned_rows(out), "ts_attn_fwd: q/out must be 16-byte aligned "
               "with strides that are multiples of 8 elements");
  TS_CHECK_ARG(lse && lse_ld >= P.q_rows, "ts_attn_fwd: lse null or lse_ld %lld < rows %lld",
               (long long)lse_ld, (long long)P.q_rows);
  const int group = P.hq / P.hkv;
  const int gc = heads_per_block(group);
  const dim3 grid((unsigned)(P.n_q_work * P.hkv * (group / gc)));
  hipStream_t s = (hipStream_t)stream;
  if (gc == 4)
    { ts::TimedLaunch timed_("attention.fwd_kernel", s); hipLaunchKernelGGL(fwd_kernel<4>, grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld); }
  else if (gc == 2)
    { ts::TimedLaunch timed_("attention.fwd_kernel", s); hipLaunchKernelGGL(fwd_kernel<2>, grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld); }
  else
    { ts::TimedLaunch timed_("attention.fwd_kernel", s); hipLaunchKernelGGL(fwd_kernel<1>, grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld); }
  return ts::check_launch("ts_attn_fwd");
}

int ts_attn_bwd(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out, ts_attn_rows dout,
                const float* lse, int64_t lse_ld, float* rowstats, ts_attn_rows dq, void* stream) {
  using namespace ts::attn;
  int st = validate(problem, "ts_attn_bwd");
  if (st != TS_OK) return st;
  const ts_attn_problem& P = *problem;
  if (P.n_q_work == 0 && P.n_kv_work == 0) return TS_OK;
  TS_CHECK_ARG(aligned_rows(q) && aligned_rows(out) && aligned_rows(dout) && aligned_rows(dq),
               "ts_attn_bwd: q/out/dout/dq must be 16-byte aligned with strides that are "
               "multiples of 8 elements");
  TS_CHECK_ARG(q.row_stride < (1ll << 25) && dout.row_stride < (1ll << 25),
               "ts_attn_bwd: q/dout row strides must be below 2^25 elements");
  TS_CHECK_ARG(lse && rowstats && lse_ld >= P.q_rows, "ts_attn_bwd: lse/rowstats null or lse_ld too small");
  TS_CHECK_ARG(P.n_kv_work == 0 || (P.kv_work && P.run_visits), "ts_attn_bwd: null kv tables");
  hipStream_t s = (hipStream_t)stream;
  const int64_t pairs = P.q_rows * P.hq;
  if (pairs > 0) {
    { ts::TimedLaunch timed_("attention.delta_kernel", s); hipLaunchKernelGGL(delta_kernel, dim3((unsigned)((pairs + 15) / 16)), dim3(kThreads), 0, s, out,
                       dout, lse, rowstats, lse_ld, P.q_rows, P.hq); }
    st = ts::check_launch("ts_attn_bwd (delta)");
    if (st != TS_OK) return st;
  }
  const int group = P.hq / P.hkv;
  const int gc = heads_per_block(group);
  if (P.n_q_work > 0) {
    const dim3 grid((unsigned)(P.n_q_work * P.hkv * (group / gc)));
    if (gc == 4)
      { ts::TimedLaunch timed_("attention.dq_kernel", s); hipLaunchKernelGGL(dq_kernel<4>, grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, dq); }
    else if (gc == 2)
      { ts::TimedLaunch timed_("attention.dq_kernel", s); hipLaunchKernelGGL(dq_kernel<2>, grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, dq); }
    else
      { ts::TimedLaunch timed_("attention.dq_kernel", s); hipLaunchKernelGGL(dq_kernel<1>, grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, dq); }
    st = ts::check_launch("ts_attn_bwd (dq)");
    if (st != TS_OK) return st;
  }
  if (P.n_kv_work > 0) {
    const dim3 grid((unsigned)(P.n_kv_work * P.hkv));
    if (group % 4 == 0) {
      { ts::TimedLaunch timed_("attention.dkdv_kernel", s); hipLaunchKernelGGL(dkdv_wave_kernel<3>, grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld); }
    } else {
      { ts::TimedLaunch timed_("attention.dkdv_kernel", s); hipLaunchKernelGGL(dkdv_kernel, grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld); }
    }
    st = ts::check_launch("ts_attn_bwd (dkdv)");
  }
  return st;
}

}  // extern "C"
