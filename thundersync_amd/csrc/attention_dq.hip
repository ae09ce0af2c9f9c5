// Attention backward: row statistics and dQ (query-stationary).
#include "attention_dq_wave.h"

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
// from ds_read_b64_tr_b16 (tr_frag).
template <typename E, int GC, int HD>
__global__ __launch_bounds__(kThreads, 1) void dq_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                         ts_attn_rows dO, const float* __restrict__ rowstats,
                                                         int64_t lse_ld, ts_attn_rows dQ) {
  constexpr int NMB = HD / 16;  // 16-column blocks of dQ
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
  f32x4 acc[2][NMB];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) acc[qb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};

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
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
          const bf16x8 kt = tr_frag<HD>(sk, 32 * ss, mb, lane);
          acc[0][mb] = mma16<E>(kt, dsk[0], acc[0][mb]);
          acc[1][mb] = mma16<E>(kt, dsk[1], acc[1][mb]);
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int row = wq0 + 16 * qb + (lane & 15);
    if (row >= T) continue;
    // acc[qb][mb] lane holds d = 16 mb + 4 g4 + i of this row: 8-byte stores
    bf16* drow = (bf16*)dQ.ptr + (seg.q_row0 + row) * dQ.row_stride + (int64_t)h * dQ.head_stride + 4 * (lane >> 4);
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const f32x4 v = acc[qb][mb] * P.scale;
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
    case 256: launch_dq_wave256(P, gc, grid, q, dout, rowstats, lse_ld, dq, s); break;
    default: {
      ts::TimedLaunch timed_("attention.dq_kernel", s);
      if (gc == 4)
        hipLaunchKernelGGL((dq_wave_kernel<E, kDqRowsPerWave / 16>), grid, dim3(64 * 128 / kDqRowsPerWave), 0, s, P, q,
                           dout, rowstats, lse_ld, dq);
      else if (gc == 2)
        hipLaunchKernelGGL((dq_wave_kernel<E, 1, D, 2>), grid, dim3(512), 0, s, P, q, dout, rowstats, lse_ld, dq);
      else
        hipLaunchKernelGGL((dq_wave_kernel<E, 1, D, 1>), grid, dim3(512), 0, s, P, q, dout, rowstats, lse_ld, dq);
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
