// Attention backward: row statistics and dQ (query-stationary).
#include "attention_impl.h"

namespace ts {
namespace attn {

// ---------------------------------------------------------------------------
// backward preprocess: per (head, row) the pair (lse * log2(e), delta) with
// delta = sum_d dO * O (fp32); a row that saw no key (lse = -inf) gets +inf
// so that exp2(s * scale * log2(e) - lse2) is 0.  The two values of a row are
// adjacent so the backward kernels fetch a tile's statistics in one load.
// ---------------------------------------------------------------------------
template <typename E, int HD>
__global__ __launch_bounds__(kThreads) void delta_kernel(ts_attn_rows O, ts_attn_rows dO,
                                                         const float* __restrict__ lse,
                                                         float* __restrict__ rowstats, int64_t lse_ld,
                                                         int64_t rows, int hq) {
  const int64_t pair = (int64_t)blockIdx.x * (kThreads / 16) + threadIdx.x / 16;
  const int sub = threadIdx.x & 15;
  const int64_t row = pair / hq;
  const int h = (int)(pair % hq);
  if (row >= rows) return;
  // 16 lanes per (row, head), HD / 16 elements each.  O is read only here
  // (non-temporal); dO stays cached for the dQ and dK/dV kernels that follow
  constexpr int PER = HD / 16;
  const bf16* op = (const bf16*)O.ptr + row * O.row_stride + (int64_t)h * O.head_stride + PER * sub;
  const bf16* dp = (const bf16*)dO.ptr + row * dO.row_stride + (int64_t)h * dO.head_stride + PER * sub;
  float acc = 0.f;
  auto add2 = [&](uint32_t a, uint32_t b) {
    acc = fmaf(bits_to_f<E>(a & 0xffffu), bits_to_f<E>(b & 0xffffu), acc);
    acc = fmaf(bits_to_f<E>(a >> 16), bits_to_f<E>(b >> 16), acc);
  };
  if constexpr (PER % 8 == 0) {
#pragma unroll
    for (int c = 0; c < PER / 8; ++c) {
      const u32x4 a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(op + 8 * c));
      const u32x4 b = ld16(dp + 8 * c);
#pragma unroll
      for (int i = 0; i < 4; ++i) add2(a[i], b[i]);
    }
  } else {
    // PER = 2, 4 or 6: 4-byte loads
#pragma unroll
    for (int c = 0; c < PER / 2; ++c)
      add2(__builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(op) + c),
           reinterpret_cast<const uint32_t*>(dp)[c]);
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
// Register-staged dQ for any supported head dim HD (the forward's work split:
// wave w takes head w % GC and rows 32 (w / GC) ..); K^T for dQ^T += K^T dS^T
// from register transposes of 8 x 8 blocks.
template <typename E, int GC, int HD>
__global__ __launch_bounds__(kThreads, 1) void dq_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                         ts_attn_rows dO, const float* __restrict__ rowstats,
                                                         int64_t lse_ld, ts_attn_rows dQ) {
  constexpr int NH = col_blocks<HD>();
  __shared__ __attribute__((aligned(16))) bf16 sk[BK * pitch_of<HD>()];
  __shared__ __attribute__((aligned(16))) bf16 sv[BK * pitch_of<HD>()];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int yb;
  const int item = task_of(P.n_q_work, P.n_q_long, yb);
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

  bf16x8 qreg[2][HD / 32], dreg[2][HD / 32];
  const int64_t qoff = (seg.q_row0 + wq0);
  load_rows_b<2, HD>(qreg, (const bf16*)Q.ptr + qoff * Q.row_stride + (int64_t)h * Q.head_stride, Q.row_stride,
                     active ? T - wq0 : 0, lane);
  load_rows_b<2, HD>(dreg, (const bf16*)dO.ptr + qoff * dO.row_stride + (int64_t)h * dO.head_stride,
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
  f32x4 acc[2][NH][8];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int hh = 0; hh < NH; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[qb][hh][e] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int sp = 0; sp < seg.nspan; ++sp) {
    const ts_attn_ref ref = load_uniform(P.seg_spans, seg.span0 + sp);
    const ts_attn_run run = load_uniform(P.runs, ref.index);
    const bf16* kb0 = (const bf16*)run.k + (int64_t)hk * run.k_head_stride;
    const bf16* vb0 = (const bf16*)run.v + (int64_t)hk * run.v_head_stride;
    for (int kt0 = 0; kt0 < run.len; kt0 += BK) {
      if (ref.kpos + kt0 > off + wg_last) break;
      const int nvalid = min(BK, run.len - kt0);
      stage_kv<HD>(sk, sv, kb0 + (int64_t)kt0 * run.k_row_stride, run.k_row_stride,
                   vb0 + (int64_t)kt0 * run.v_row_stride, run.v_row_stride, nvalid, tid);
      if (!active || ref.kpos + kt0 > off + w_last) continue;

      f32x4 s[4][2], dp[4][2];
      tile_scores<E, HD>(s, sk, qreg, lane);
      tile_scores<E, HD>(dp, sv, dreg, lane);  // dP^T = V dO^T, same shape as S^T
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
          dsk[qb] = pack8<E>(tmp);
        }
        int rows[8];
        slot_rows(lane >> 4, 32 * ss, rows);
#pragma unroll
        for (int hh = 0; hh < NH; ++hh) {
          bf16x8 kt[8];
          lds_rows_transposed<HD>(sk, rows, col_start<HD>(hh, lane), kt);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            acc[0][hh][e] = mma16<E>(kt[e], dsk[0], acc[0][hh][e]);
            acc[1][hh][e] = mma16<E>(kt[e], dsk[1], acc[1][hh][e]);
          }
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
    for (int hh = 0; hh < NH; ++hh)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (!col_valid<HD>(hh, lane >> 4, i)) continue;
        float tmp[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) tmp[e] = acc[qb][hh][e][i] * P.scale;
        st16(drow + 128 * hh + 8 * i, as_u32x4(pack8<E>(tmp)));
      }
  }
}

// ---------------------------------------------------------------------------
// backward dQ for GQA groups that are a multiple of 4 (query-stationary)
//
// A work-group owns 32 query rows of one segment for the 4 query heads of one
// quarter of a GQA group; wave w takes head w & 3 and 16 NQB of the rows
// (NQB = 1: eight waves, two per SIMD, so that one wave's LDS and MFMA waits
// are covered by the other's work; NQB = 2: four waves of 32 rows, one per
// SIMD).  Q and dO rows stay in registers as B operands, with the rows'
// (lse * log2 e, delta) pairs.  The segment's key runs stream through 64-key
// K/V tiles that all waves share: double-buffered LDS stages filled by
// buffer_load ... lds (each wave issues its share of a tile's instructions;
// rows past a run's end arrive as zeros and add nothing, because a zero K row
// contributes zero to dQ), one work-group barrier per tile.  Tiles use the dK/dV kernel's 256-byte rows
// with chunk c of row r at slot c ^ tile_swizzle(r & 15): K and V rows feed S^T = K Q^T
// and dP^T = V dO^T as A operands, K^T for dQ^T += K^T dS^T comes from
// ds_read_b64_tr_b16.  Only tiles that cross the diagonal are masked.
// ---------------------------------------------------------------------------
template <typename E, int NQB>
__global__ __launch_bounds__(64 * 8 / NQB, 1) void dq_wave_kernel(ts_attn_problem P, ts_attn_rows Q, ts_attn_rows dO,
                                                                 const float* __restrict__ rowstats,
                                                                 int64_t lse_ld, ts_attn_rows dQ) {
  constexpr int kWaves = 8 / NQB;
  __shared__ __attribute__((aligned(16))) bf16 s_k0[kKV64];
  __shared__ __attribute__((aligned(16))) bf16 s_v0[kKV64];
  __shared__ __attribute__((aligned(16))) bf16 s_k1[kKV64];
  __shared__ __attribute__((aligned(16))) bf16 s_v1[kKV64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, j16 = lane & 15;
  int yb;
  const int item = task_of(P.n_q_work, P.n_q_long, yb);
  const int seg_id = uniform_table(P.q_work)[2 * item];
  const int q0 = uniform_table(P.q_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const int chunks = group / 4;
  const int hk = yb / chunks;
  const int h = hk * group + (yb % chunks) * 4 + (wave & 3);
  const int qw = q0 + 16 * NQB * (wave >> 2);  // this wave's first row
  const ts_attn_segment seg = load_uniform(P.segs, seg_id);
  const int T = seg.q_len;
  const int off = seg.kv_len - seg.q_len;
  const int last = min(q0 + 32, T) - 1;
  const float c = P.scale * kLog2e;

  // Q / dO rows as B operands: reg[qb][ks] = row qw + 16 qb + j16, columns 32 ks + 8 g4 ..
  bf16x8 qreg[NQB][4], dreg[NQB][4];
  const int64_t row0 = seg.q_row0 + qw;
  load_rows_b(qreg, (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)h * Q.head_stride, Q.row_stride,
              T - qw, lane);
  load_rows_b(dreg, (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)h * dO.head_stride,
              dO.row_stride, T - qw, lane);
  // rows past the segment: zero Q and dO with statistics (0, 0) give dS = 0
  float lse2[NQB], dlt[NQB];
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int row = qw + 16 * qb + j16;
    lse2[qb] = 0.f;
    dlt[qb] = 0.f;
    if (row < T) {
      const int64_t at = 2 * ((int64_t)h * lse_ld + seg.q_row0 + row);
      lse2[qb] = rowstats[at];
      dlt[qb] = rowstats[at + 1];
    }
  }
  f32x4 ndlt[NQB];  // -delta of the lane's row, the starting value of the dP^T accumulators
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) ndlt[qb] = f32x4{-dlt[qb], -dlt[qb], -dlt[qb], -dlt[qb]};
  f32x4 acc[8][NQB];
#pragma unroll
  for (int mb = 0; mb < 8; ++mb)
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) acc[mb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};

  int ro[4], to[8];
  swizzled_offsets(lane, ro, to);

  // one 32-key half ss of a tile: S^T = K Q^T, dP^T = V dO^T for keys
  // 32 ss .. 32 ss + 31 ([kb][qb] lane holds keys 32 ss + 16 kb + 4 g4 + i,
  // row 16 qb + j16)
  auto scores = [&](const bf16* tk, const bf16* tv, int ss, f32x4 (&sc)[2][NQB], f32x4 (&dp)[2][NQB])
      __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        sc[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[kb][qb] = ndlt[qb];  // the MFMAs accumulate dP^T - delta
      }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 ak = as_bf16x8(ld16(tk + ro[ks] + (32 * ss + 16 * kb) * D));
        const bf16x8 av = as_bf16x8(ld16(tv + ro[ks] + (32 * ss + 16 * kb) * D));
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          sc[kb][qb] = mma16<E>(ak, qreg[qb][ks], sc[kb][qb]);
          dp[kb][qb] = mma16<E>(av, dreg[qb][ks], dp[kb][qb]);
        }
      }
  };
  // dS^T = P^T (dP^T - delta) (dp holds dP^T - delta), P^T = exp2(S^T c - lse2), packed as the B
  // operand of dQ^T += K^T dS^T (slot j <-> key 32 ss + 16 (j >> 2) + 4 g4 +
  // (j & 3)); DIAG masks keys past each row's diagonal
  auto dscores = [&](auto diag, int kpos, int kt0, int ss, f32x4 (&sc)[2][NQB], const f32x4 (&dp)[2][NQB],
                     bf16x8 (&dsk)[NQB]) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        // row qw + 16 qb + j16 sees key kt0 + 32 ss + 16 kb + 4 g4 + i iff i <= lim
        const int lim = off + qw + 16 * qb + j16 - kpos - kt0 - 32 * ss - 16 * kb - 4 * g4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float p = fast_exp2(sc[kb][qb][i] * c - lse2[qb]);
          if (decltype(diag)::value) p = i <= lim ? p : 0.f;
          sc[kb][qb][i] = p * dp[kb][qb][i];
        }
      }
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) {
      float tmp[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) tmp[j] = sc[j >> 2][qb][j & 3];
      dsk[qb] = pack8<E>(tmp);
    }
  };
  auto accumulate = [&](const bf16* tk, int ss, const bf16x8 (&dsk)[NQB]) __attribute__((always_inline)) {
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const u32x2 a0 = tr_read(tk + to[mb] + 32 * ss * D);
      const u32x2 a1 = tr_read(tk + to[mb] + (32 * ss + 16) * D);
      const bf16x8 a = as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) acc[mb][qb] = mma16<E>(a, dsk[qb], acc[mb][qb]);
    }
  };
  // one tile, the halves software-pipelined: half 1's score MFMAs are issued
  // beside half 0's exponentials, half 0's dQ MFMAs beside half 1's
  auto tile_body = [&](auto diag, const bf16* tk, const bf16* tv, int kpos, int kt0) __attribute__((always_inline)) {
    f32x4 sc0[2][NQB], dp0[2][NQB], sc1[2][NQB], dp1[2][NQB];
    bf16x8 dsk0[NQB], dsk1[NQB];
    scores(tk, tv, 0, sc0, dp0);
    __builtin_amdgcn_sched_barrier(0);
    scores(tk, tv, 1, sc1, dp1);
    dscores(diag, kpos, kt0, 0, sc0, dp0, dsk0);
    // 16 K/V reads and 16 NQB MFMAs of half 1 beside ~40 NQB VALU instructions
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // the first K/V reads of half 1
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NQB, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, NQB == 2 ? 5 : 3, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, NQB, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, NQB == 2 ? 4 : 3, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    dscores(diag, kpos, kt0, 1, sc1, dp1, dsk1);
    accumulate(tk, 0, dsk0);
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);  // K^T reads for dQ of half 0
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x002, NQB == 2 ? 4 : 5, 1);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    accumulate(tk, 1, dsk1);
    // K^T fragment reads of half 1 kept four blocks ahead of their MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 2);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      __builtin_amdgcn_sched_group_barrier(0x008, NQB, 2);
      if (mb + 4 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 2, 2);
    }
  };

  auto step = [&](auto bsel, TileCursor& cur) {
    const int kpos = cur.kpos;
    const int kt0 = cur.kt0;
    const TileCursor nxt = next_kv_tile(P, seg, last, cur);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the tile has landed
    __syncthreads();                // every part has, and the other stage is free
    const bf16* tk = bsel.value == 0 ? s_k0 : s_k1;
    const bf16* tv = bsel.value == 0 ? s_v0 : s_v1;
    if (nxt.sp < seg.nspan)
      issue_kv_tile<kWaves>(hk, wave, lane, nxt, bsel.value == 0 ? s_k1 : s_k0, bsel.value == 0 ? s_v1 : s_v0);

    if (kpos + kt0 + BK - 1 > off + qw)
      tile_body(std::true_type{}, tk, tv, kpos, kt0);
    else
      tile_body(std::false_type{}, tk, tv, kpos, kt0);
    cur = nxt;
  };

  TileCursor cur = first_kv_tile(P, seg, last);
  if (cur.sp < seg.nspan) issue_kv_tile<kWaves>(hk, wave, lane, cur, s_k0, s_v0);
  while (cur.sp < seg.nspan) {
    step(std::integral_constant<int, 0>{}, cur);
    if (cur.sp >= seg.nspan) break;
    step(std::integral_constant<int, 1>{}, cur);
  }

  // dQ^T: acc[mb][qb] lane holds d = 16 mb + 4 g4 + i of row qw + 16 qb + j16
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int row = qw + 16 * qb + j16;
    if (row >= T) continue;
    bf16* drow = (bf16*)dQ.ptr + (seg.q_row0 + row) * dQ.row_stride + (int64_t)h * dQ.head_stride + 4 * g4;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const f32x4 v = acc[mb][qb] * P.scale;
      *reinterpret_cast<u32x2*>(drow + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    }
  }
}

template <typename E, int HD>
void launch_delta_hd(const ts_attn_problem& P, ts_attn_rows out, ts_attn_rows dout, const float* lse, float* rowstats,
                     int64_t lse_ld, int64_t pairs, hipStream_t s) {
  ts::TimedLaunch timed_("attention.delta_kernel", s);
  hipLaunchKernelGGL((delta_kernel<E, HD>), dim3((unsigned)((pairs + 15) / 16)), dim3(kThreads), 0, s, out, dout, lse,
                     rowstats, lse_ld, P.q_rows, P.hq);
}

template <typename E>
int launch_delta_t(const ts_attn_problem& P, ts_attn_rows out, ts_attn_rows dout, const float* lse,
                 float* rowstats, int64_t lse_ld, hipStream_t s) {
  const int64_t pairs = P.q_rows * P.hq;
  if (pairs == 0) return TS_OK;
  switch (P.head_dim) {
    case 32: launch_delta_hd<E, 32>(P, out, dout, lse, rowstats, lse_ld, pairs, s); break;
    case 64: launch_delta_hd<E, 64>(P, out, dout, lse, rowstats, lse_ld, pairs, s); break;
    case 96: launch_delta_hd<E, 96>(P, out, dout, lse, rowstats, lse_ld, pairs, s); break;
    case 192: launch_delta_hd<E, 192>(P, out, dout, lse, rowstats, lse_ld, pairs, s); break;
    case 256: launch_delta_hd<E, 256>(P, out, dout, lse, rowstats, lse_ld, pairs, s); break;
    default: launch_delta_hd<E, D>(P, out, dout, lse, rowstats, lse_ld, pairs, s);
  }
  return ts::check_launch("ts_attn_bwd (delta)");
}

// query rows per wave of the dQ kernel (16: eight waves, two per SIMD; 32: four)
constexpr int kDqRowsPerWave = 16;

template <typename E, int HD>
void launch_dq_generic(const ts_attn_problem& P, int gc, dim3 grid, ts_attn_rows q, ts_attn_rows dout,
                       const float* rowstats, int64_t lse_ld, ts_attn_rows dq, hipStream_t s) {
  ts::TimedLaunch timed_("attention.dq_kernel", s);
  if constexpr (HD != D) {
    if (gc == 4) {
      hipLaunchKernelGGL((dq_kernel<E, 4, HD>), grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, dq);
      return;
    }
  }
  if (gc == 2)
    hipLaunchKernelGGL((dq_kernel<E, 2, HD>), grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, dq);
  else
    hipLaunchKernelGGL((dq_kernel<E, 1, HD>), grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, dq);
}

template <typename E>
int launch_dq_t(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout, const float* rowstats,
              int64_t lse_ld, ts_attn_rows dq, hipStream_t s) {
  const int group = P.hq / P.hkv;
  const int gc = heads_per_block(group);
  const dim3 grid((unsigned)(P.n_q_work * P.hkv * (group / gc)));
  switch (P.head_dim) {
    case 32: launch_dq_generic<E, 32>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s); break;
    case 64: launch_dq_generic<E, 64>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s); break;
    case 96: launch_dq_generic<E, 96>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s); break;
    case 192: launch_dq_generic<E, 192>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s); break;
    case 256: launch_dq_generic<E, 256>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s); break;
    default:
      if (gc == 4) {
        ts::TimedLaunch timed_("attention.dq_kernel", s);
        hipLaunchKernelGGL((dq_wave_kernel<E, kDqRowsPerWave / 16>), grid, dim3(64 * 128 / kDqRowsPerWave), 0, s, P, q,
                           dout, rowstats, lse_ld, dq);
      } else {
        launch_dq_generic<E, D>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s);
      }
  }
  return ts::check_launch("ts_attn_bwd (dq)");
}

int launch_delta(const ts_attn_problem& P, ts_attn_rows out, ts_attn_rows dout, const float* lse,
                 float* rowstats, int64_t lse_ld, hipStream_t s) {
  return P.dtype == kF16 ? launch_delta_t<f16>(P, out, dout, lse, rowstats, lse_ld, s)
                         : launch_delta_t<bf16>(P, out, dout, lse, rowstats, lse_ld, s);
}

int launch_dq(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout, const float* rowstats,
              int64_t lse_ld, ts_attn_rows dq, hipStream_t s) {
  return P.dtype == kF16 ? launch_dq_t<f16>(P, q, dout, rowstats, lse_ld, dq, s)
                         : launch_dq_t<bf16>(P, q, dout, rowstats, lse_ld, dq, s);
}

}  // namespace attn
}  // namespace ts
