// The dQ kernel that shares K/V tiles among its waves, as a template: compiled
// at head dim 128 in attention_dq.hip (MFMA results in VGPRs) and at head dim
// 256 in attention_dq256.hip (MFMA results in the accumulation registers: four
// waves of 32 rows need more than the 256 VGPRs for their dQ accumulators).
#pragma once
#include "attention_impl.h"

namespace ts {
namespace attn {

// ---------------------------------------------------------------------------
// backward dQ with the waves sharing K/V tiles (query-stationary; head dim 128
// with GQA groups that are a multiple of 4 (GC = 4), head dim 256 with any
// group, GC heads per work-group)
//
// A work-group owns 128 / GC query rows of one segment for GC query heads of
// one GQA group; wave w takes head w % GC and 16 NQB of the rows (head dim
// 128: NQB = 1, eight waves, two per SIMD, so that one wave's LDS and MFMA
// waits are covered by the other's work; head dim 256: NQB = 2, four waves of
// 32 rows, one per SIMD).  Q and dO rows stay in registers as B operands, with
// the rows' (lse * log2 e, delta) pairs.  The segment's key runs stream
// through 64-key K/V tiles that all waves share: double-buffered LDS stages
// filled by buffer_load ... lds (each wave issues its share of a tile's
// instructions; rows past a run's end arrive as zeros and add nothing,
// because a zero K row contributes zero to dQ), one work-group barrier per
// tile.  Tiles use the dK/dV kernel's swizzled rows
// with chunk c of row r at slot c ^ tile_swizzle(r & 15): K and V rows feed S^T = K Q^T
// and dP^T = V dO^T as A operands, K^T for dQ^T += K^T dS^T comes from
// ds_read_b64_tr_b16.  Only tiles that cross the diagonal are masked.
// ---------------------------------------------------------------------------
template <typename E, int NQB, int HD = D, int GC = 4, int NP = 1>
__global__ __launch_bounds__(64 * 8 / (NQB * NP), 1) void dq_wave_kernel(ts_attn_problem P, ts_attn_rows Q, ts_attn_rows dO,
                                                                 const float* __restrict__ rowstats,
                                                                 int64_t lse_ld, ts_attn_rows dQ) {
  constexpr int kWaves = 8 / (NQB * NP);
  constexpr int kPassRows = 16 * NQB * kWaves / GC;  // rows of the work item one pass covers
  constexpr int NKS = HD / 32, NMB = HD / 16;  // k-steps of S / dP; 16-column blocks of dQ
  __shared__ __attribute__((aligned(16))) bf16 s_k0[BK * HD];
  __shared__ __attribute__((aligned(16))) bf16 s_v0[BK * HD];
  __shared__ __attribute__((aligned(16))) bf16 s_k1[BK * HD];
  __shared__ __attribute__((aligned(16))) bf16 s_v1[BK * HD];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, j16 = lane & 15;
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
  const float c = P.scale * kLog2e;
  int ro[4], to[8];
  swizzled_offsets<HD>(lane, ro, to);

  // the work item's rows in NP passes over its keys (one at head dim 128)
#pragma unroll 1
  for (int pass = 0; pass < NP; ++pass) {
  const int qp = q0 + pass * kPassRows;  // the pass's first row
  if constexpr (NP > 1) {
    if (qp >= T) break;
    __builtin_amdgcn_s_waitcnt(0);  // the previous pass's last (empty) DMA has landed
    __syncthreads();                // and no wave still reads its stages
  }
  const int qw = qp + 16 * NQB * (wave / GC);  // this wave's first row
  const int last = min(qp + kPassRows, T) - 1;
  // Q / dO rows as B operands: reg[qb][ks] = row qw + 16 qb + j16, columns 32 ks + 8 g4 ..
  bf16x8 qreg[NQB][NKS], dreg[NQB][NKS];
  const int64_t row0 = seg.q_row0 + qw;
  load_rows_b<NQB, HD>(qreg, (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)h * Q.head_stride, Q.row_stride,
              T - qw, lane);
  load_rows_b<NQB, HD>(dreg, (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)h * dO.head_stride,
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
  f32x4 acc[NMB][NQB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
    for (int qb = 0; qb < NQB; ++qb) acc[mb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};

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
      for (int ks = 0; ks < NKS; ++ks) {
        const bf16x8 ak = as_bf16x8(ld16(tk + ro_of(ro, ks) + (32 * ss + 16 * kb) * HD));
        const bf16x8 av = as_bf16x8(ld16(tv + ro_of(ro, ks) + (32 * ss + 16 * kb) * HD));
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
    for (int mb = 0; mb < NMB; ++mb) {
      const u32x2 a0 = tr_read(tk + to_of(to, mb) + 32 * ss * HD);
      const u32x2 a1 = tr_read(tk + to_of(to, mb) + (32 * ss + 16) * HD);
      const bf16x8 a = as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) acc[mb][qb] = mma16<E>(a, dsk[qb], acc[mb][qb]);
    }
  };
  // one tile, the halves software-pipelined: half 1's score MFMAs are issued
  // beside half 0's exponentials, half 0's dQ MFMAs beside half 1's
  auto tile_body = [&](auto diag, const bf16* tk, const bf16* tv, int kpos, int kt0) __attribute__((always_inline)) {
    if constexpr (HD > 128 && kWaves == 8) {
      // at head dim 256 with two waves per SIMD the halves run one after the
      // other: the pipelined form's two halves of S and dP do not fit the
      // registers beside the dQ accumulators and the Q/dO rows
#pragma unroll
      for (int ss = 0; ss < 2; ++ss) {
        f32x4 sc[2][NQB], dp[2][NQB];
        bf16x8 dsk[NQB];
        scores(tk, tv, ss, sc, dp);
        // K/V row reads two (kb, ks) steps ahead of their MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 3);
#pragma unroll
        for (int i = 0; i < 2 * NKS; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 2 * NQB, 3);
          if (i + 2 < 2 * NKS) __builtin_amdgcn_sched_group_barrier(0x100, 2, 3);
        }
        __builtin_amdgcn_sched_barrier(0);
        dscores(diag, kpos, kt0, ss, sc, dp, dsk);
        accumulate(tk, ss, dsk);
        // K^T fragment reads kept four blocks ahead of their MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 4);
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
          __builtin_amdgcn_sched_group_barrier(0x008, NQB, 4);
          if (mb + 4 < NMB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 4);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
    f32x4 sc0[2][NQB], dp0[2][NQB], sc1[2][NQB], dp1[2][NQB];
    bf16x8 dsk0[NQB], dsk1[NQB];
    scores(tk, tv, 0, sc0, dp0);
    __builtin_amdgcn_sched_barrier(0);
    scores(tk, tv, 1, sc1, dp1);
    dscores(diag, kpos, kt0, 0, sc0, dp0, dsk0);
    // 4 NKS K/V reads and 4 NKS NQB MFMAs of half 1 beside ~40 NQB VALU instructions
    constexpr int v1 = (NQB == 2 ? 5 : 3) * 4 / NKS > 0 ? (NQB == 2 ? 5 : 3) * 4 / NKS : 1;
    constexpr int v2 = (NQB == 2 ? 4 : 3) * 4 / NKS > 0 ? (NQB == 2 ? 4 : 3) * 4 / NKS : 1;
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // the first K/V reads of half 1
#pragma unroll
    for (int i = 0; i < 4 * NKS - 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, NQB, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, v1, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, NQB, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, v2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    dscores(diag, kpos, kt0, 1, sc1, dp1, dsk1);
    accumulate(tk, 0, dsk0);
    constexpr int v3 = (NQB == 2 ? 4 : 5) * 8 / NMB > 0 ? (NQB == 2 ? 4 : 5) * 8 / NMB : 1;
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 1);  // K^T reads for dQ of half 0
#pragma unroll
    for (int i = 0; i < NMB; ++i) {
      if (i < NMB - 8)
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
      else
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x002, v3, 1);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    accumulate(tk, 1, dsk1);
    // K^T fragment reads of half 1 kept four blocks ahead of their MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 2);
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      __builtin_amdgcn_sched_group_barrier(0x008, NQB, 2);
      if (mb + 4 < NMB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 2);
    }
  };

  auto step = [&](auto bsel, TileCursor& cur) {
    const int kpos = cur.kpos;
    const int kt0 = cur.kt0;
    const TileCursor nxt = next_kv_tile(P, seg, hk, last, cur);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the tile has landed
    __syncthreads();                // every part has, and the other stage is free
    const bf16* tk = bsel.value == 0 ? s_k0 : s_k1;
    const bf16* tv = bsel.value == 0 ? s_v0 : s_v1;
    if (nxt.sp < seg.nspan)
      issue_kv_tile<kWaves, HD>(wave, lane, nxt, bsel.value == 0 ? s_k1 : s_k0, bsel.value == 0 ? s_v1 : s_v0);

    if (kpos + kt0 + BK - 1 > off + qw)
      tile_body(std::true_type{}, tk, tv, kpos, kt0);
    else
      tile_body(std::false_type{}, tk, tv, kpos, kt0);
    cur = nxt;
  };

  TileCursor cur = first_kv_tile(P, seg, hk, last);
  if (cur.sp < seg.nspan) issue_kv_tile<kWaves, HD>(wave, lane, cur, s_k0, s_v0);
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
    for (int mb = 0; mb < NMB; ++mb) {
      const f32x4 v = acc[mb][qb] * P.scale;
      *reinterpret_cast<u32x2*>(drow + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    }
  }
  }
}


// dQ at head dim 256 (attention_dq256.hip): the one-wave-per-SIMD instance
void launch_dq_wave256(const ts_attn_problem& P, int gc, dim3 grid, ts_attn_rows q, ts_attn_rows dout,
                       const float* rowstats, int64_t lse_ld, ts_attn_rows dq, hipStream_t s);

}  // namespace attn
}  // namespace ts
