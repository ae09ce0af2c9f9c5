// Attention forward kernel (query-stationary online softmax).
#include "attention_impl.h"

namespace ts {
namespace attn {

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

int launch_fwd(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows out, float* lse, int64_t lse_ld,
               hipStream_t s) {
  const int group = P.hq / P.hkv;
  const int gc = heads_per_block(group);
  const dim3 grid((unsigned)(P.n_q_work * P.hkv * (group / gc)));
  if (gc == 4)
    { ts::TimedLaunch timed_("attention.fwd_kernel", s); hipLaunchKernelGGL(fwd_kernel<4>, grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld); }
  else if (gc == 2)
    { ts::TimedLaunch timed_("attention.fwd_kernel", s); hipLaunchKernelGGL(fwd_kernel<2>, grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld); }
  else
    { ts::TimedLaunch timed_("attention.fwd_kernel", s); hipLaunchKernelGGL(fwd_kernel<1>, grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld); }
  return ts::check_launch("ts_attn_fwd");
}

}  // namespace attn
}  // namespace ts
