// Attention forward kernel (query-stationary online softmax).
#include "attention_impl.h"

namespace ts {
namespace attn {

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// Register-staged forward for any supported head dim HD and GQA groups that
// are not a multiple of 4 (and, at head dims other than 128, those that are):
// a work-group owns 32 4 / GC query rows of GC query heads (wave w: head
// w % GC, rows 32 (w / GC) ..); K/V tiles of 64 keys pass through registers
// into padded LDS rows; V^T comes from ds_read_b64_tr_b16 (tr_frag).
template <typename E, int GC, int HD>
__global__ __launch_bounds__(kThreads, HD > 128 ? 1 : 2) void fwd_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                          ts_attn_rows O, float* __restrict__ lse,
                                                          int64_t lse_ld) {
  constexpr int NMB = HD / 16;  // 16-column blocks of O
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

  bf16x8 qreg[2][HD / 32];
  const bf16* qbase = (const bf16*)Q.ptr + (seg.q_row0 + wq0) * Q.row_stride + (int64_t)h * Q.head_stride;
  load_rows_b<2, HD>(qreg, qbase, Q.row_stride, active ? T - wq0 : 0, lane);

  f32x4 o[2][NMB];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) o[qb][mb] = f32x4{0.f, 0.f, 0.f, 0.f};
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
      stage_kv<HD>(sk, sv, kb0 + (int64_t)kt0 * run.k_row_stride, run.k_row_stride,
                   vb0 + (int64_t)kt0 * run.v_row_stride, run.v_row_stride, nvalid, tid);
      if (!active || ref.kpos + kt0 > off + w_last) continue;

      f32x4 s[4][2];
      tile_scores<E, HD>(s, sk, qreg, lane);
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
        mx = rows_max4(mx);
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
        for (int mb = 0; mb < NMB; ++mb) o[qb][mb] *= alpha;
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
          pk[qb] = pack8<E>(tmp);
        }
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
          const bf16x8 vt = tr_frag<HD>(sv, 32 * ss, mb, lane);
          o[0][mb] = mma16<E>(vt, pk[0], o[0][mb]);
          o[1][mb] = mma16<E>(vt, pk[1], o[1][mb]);
        }
      }
    }
  }
  if (!active) return;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float l = rows_sum4(lsum[qb]);
    const int row = wq0 + 16 * qb + (lane & 15);
    if (row >= T) continue;
    const float inv = l > 0.f ? 1.f / l : 0.f;
    // o[qb][mb] lane holds d = 16 mb + 4 g4 + i of this row: 8-byte stores
    bf16* orow = (bf16*)O.ptr + (seg.q_row0 + row) * O.row_stride + (int64_t)h * O.head_stride + 4 * (lane >> 4);
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const f32x4 v = o[qb][mb] * inv;
      *reinterpret_cast<u32x2*>(orow + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    }
    if ((lane >> 4) == 0)
      lse[(int64_t)h * lse_ld + seg.q_row0 + row] = l > 0.f ? (m[qb] + fast_log2(l)) * kLn2 : neg_inf();
  }
}

// ---------------------------------------------------------------------------
// forward with the waves sharing K/V tiles (head dim 128 with GQA groups that
// are a multiple of 4 (GC = 4); head dim 256 with any group, GC heads per
// work-group)
//
// A work-group owns 128 / GC query rows of one segment for GC query heads of
// one GQA group; wave w takes head w % GC and 16 NQB rows (at head dim 128
// with GC = 4: NQB = 2, four waves; NQB = 1, eight waves of 16 rows, four
// waves per SIMD, measured no faster on C2 at 1.32 ms; at head dim 256
// NQB = 1, eight waves, two per SIMD, one work-group per CU for its 128 KB of
// tiles).  The heads share K/V tiles of KT keys (32 at head dim 128: 32 KB
// of stages per work-group, three work-groups and three waves per SIMD at 168
// VGPRs, against two with 64-key tiles: C2 forward 1.20 -> 1.09 ms; 64 at
// 256), streamed by buffer DMA into double-buffered swizzled LDS stages (one
// work-group barrier per tile).  Q rows stay in registers as B operands of
// S^T = K Q^T; V^T for O^T += V^T P^T comes from ds_read_b64_tr_b16.  Per 32
// keys of a tile each lane owns one query column (16 qb + j16) and 8 of the
// keys, the others sitting in the lanes j16 + 16, + 32, + 48.  The softmax runs in the
// log2 domain with the scale folded into one FMA per score, and the
// reference point m of a row moves only when the row maximum exceeds it by
// more than 8 (a factor of 256): the accumulators are rescaled in the rare
// tile where that happens (skipped wave-wide otherwise), and since O and the
// row sum share the same m the result is unchanged.  Only tiles that cross
// the diagonal or pass a run's end are masked.
// ---------------------------------------------------------------------------
constexpr float kRescaleSlack = 8.f;    // log2 units
constexpr float kRescaleBound = 256.f;  // 2^kRescaleSlack

#ifndef TS_FWD_KT128
#define TS_FWD_KT128 32
#endif
// keys per K/V tile at head dim 128 for GQA groups that are not a multiple of 4
#ifndef TS_FWD_KT128_GC
#define TS_FWD_KT128_GC 32
#endif
// work-groups per CU: their LDS stages (two K/V stages of KT keys) and registers
template <int NQB, int HD, int KT>
constexpr int fwd_occupancy() { return HD > 128 ? (NQB == 1 ? 2 : 1) : (NQB == 1 ? 4 : (KT == 32 ? 3 : 2)); }

template <typename E, int NQB, int HD = D, int GC = 4, int KT = BK>
__global__ __launch_bounds__(64 * 8 / NQB, (fwd_occupancy<NQB, HD, KT>())) void fwd_wave_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                                                  ts_attn_rows O,
                                                                                  float* __restrict__ lse,
                                                                                  int64_t lse_ld) {
  constexpr int kWaves = 8 / NQB;
  constexpr int NKS = HD / 32, NMB = HD / 16;  // k-steps of S; 16-column blocks of O
  static_assert(KT == 64 || KT == 32, "tiles of 64 or 32 keys");
  __shared__ __attribute__((aligned(16))) bf16 s_k0[KT * HD];
  __shared__ __attribute__((aligned(16))) bf16 s_v0[KT * HD];
  __shared__ __attribute__((aligned(16))) bf16 s_k1[KT * HD];
  __shared__ __attribute__((aligned(16))) bf16 s_v1[KT * HD];
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
  const int qw = q0 + 16 * NQB * (wave / GC);  // this wave's first row
  const ts_attn_segment seg = load_uniform(P.segs, seg_id);
  const int T = seg.q_len;
  const int off = seg.kv_len - seg.q_len;
  const int last = min(q0 + 16 * NQB * kWaves / GC, T) - 1;
  const float c = P.scale * kLog2e;

  // Q rows as B operands: qreg[qb][ks] = row qw + 16 qb + j16, columns 32 ks + 8 g4 ..
  bf16x8 qreg[NQB][NKS];
  load_rows_b<NQB, HD>(qreg, (const bf16*)Q.ptr + (seg.q_row0 + qw) * Q.row_stride + (int64_t)h * Q.head_stride,
              Q.row_stride, T - qw, lane);
  f32x4 acc[NMB][NQB];
  float m[NQB], l[NQB];  // reference point (log2 units) of this lane's column; its part of the
                         // column's sum of exp2(s c - m)
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) acc[mb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[qb] = neg_inf();
    l[qb] = 0.f;
  }
  int ro[4], to[8];
  swizzled_offsets<HD>(lane, ro, to);

  auto step = [&](auto bsel, TileCursor& cur) {
    const int kpos = cur.kpos, run_len = cur.len;
    const int kt0 = cur.kt0;
    const TileCursor nxt = next_kv_tile<KT>(P, seg, hk, last, cur);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's part of the tile has landed
    __syncthreads();                // every part has, and the other stage is free
    const bf16* tk = bsel.value == 0 ? s_k0 : s_k1;
    const bf16* tv = bsel.value == 0 ? s_v0 : s_v1;
    if (nxt.sp < seg.nspan)
      issue_kv_tile<kWaves, HD, KT>(wave, lane, nxt, bsel.value == 0 ? s_k1 : s_k0, bsel.value == 0 ? s_v1 : s_v0);

    const bool masked = (kpos + kt0 + KT - 1 > off + qw) | (kt0 + KT > run_len);
    // two halves of 32 keys, each one online-softmax update:
    // S^T = K Q^T with sc[kb][qb] holding keys 32 ss + 16 kb + 4 g4 + i of column
    // 16 qb + j16, then O^T += V^T P^T with slot j <-> key 32 ss + 16 (j >> 2) + 4 g4 + (j & 3)
#pragma unroll
    for (int ss = 0; ss < KT / 32; ++ss) {
      f32x4 sc[2][NQB];
      // wave priority 1 over the MFMA phases, 0 over the softmax: of the two
      // waves on a SIMD, the one with MFMAs to issue goes first (fwd -1.4 %)
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) sc[kb][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          const bf16x8 ak = as_bf16x8(ld16(tk + ro_of(ro, ks) + (32 * ss + 16 * kb) * HD));
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) sc[kb][qb] = mma16<E>(ak, qreg[qb][ks], sc[kb][qb]);
        }
      }
      // K fragment reads three (kb, ks) steps ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 1);
#pragma unroll
      for (int st = 0; st < 2 * NKS; ++st) {
        __builtin_amdgcn_sched_group_barrier(0x008, NQB, 1);
        if (st + 3 < 2 * NKS) __builtin_amdgcn_sched_group_barrier(0x100, 1, 1);
      }
      __builtin_amdgcn_s_setprio(0);
      if (masked) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < NQB; ++qb) {
            const int key0 = kt0 + 32 * ss + 16 * kb + 4 * g4;  // key of element i = key0 + i
            const int lim = min(off + qw + 16 * qb + j16 - kpos, run_len - 1) - key0;
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (i > lim) sc[kb][qb][i] = neg_inf();
          }
      }
      // Fast path: the exponentials against the current reference point m.
      // They stand unless some score exceeds m by more than kRescaleSlack, which
      // a lane detects as a partial sum above 2^kRescaleSlack (every term is
      // positive), or m is still -inf; then, rarely, the half is redone on the
      // slow path: column maxima, the move of m with the rescale of O and the
      // row sum, and the exponentials again.
      float pe[2][NQB][4], ps[NQB];
      bool redo = false;
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        const float mref = m[qb] == neg_inf() ? 0.f : m[qb];
        ps[qb] = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            pe[kb][qb][i] = fast_exp2(fmaf(sc[kb][qb][i], c, -mref));
            ps[qb] += pe[kb][qb][i];
          }
        redo |= (m[qb] == neg_inf()) | (ps[qb] > kRescaleBound);
      }
      if (__builtin_amdgcn_ballot_w64(redo) != 0) {
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) {
          float mx = fmaxf(fmaxf(fmaxf(sc[0][qb][0], sc[0][qb][1]), fmaxf(sc[0][qb][2], sc[0][qb][3])),
                           fmaxf(fmaxf(sc[1][qb][0], sc[1][qb][1]), fmaxf(sc[1][qb][2], sc[1][qb][3])));
          mx = rows_max4(mx);
          const float mt = mx * c;  // maximum in log2 units (-inf if the column sees none of these keys)
          const bool move = mt > m[qb] + kRescaleSlack;
          if (__builtin_amdgcn_ballot_w64(move) != 0) {
            const float mnew = move ? mt : m[qb];
            const float alpha = fast_exp2(m[qb] - mnew);  // 0 on the first visible keys (m = -inf)
            l[qb] *= alpha;
#pragma unroll
            for (int mb = 0; mb < NMB; ++mb) acc[mb][qb] *= alpha;
            m[qb] = mnew;
          }
          const float mref = m[qb] == neg_inf() ? 0.f : m[qb];
          ps[qb] = 0.f;
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              pe[kb][qb][i] = fast_exp2(fmaf(sc[kb][qb][i], c, -mref));
              ps[qb] += pe[kb][qb][i];
            }
        }
      }
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) l[qb] += ps[qb];
      bf16x8 pk[NQB];
#pragma unroll
      for (int qb = 0; qb < NQB; ++qb) {
        float tmp[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) tmp[j] = pe[j >> 2][qb][j & 3];
        pk[qb] = pack8<E>(tmp);
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const u32x2 a0 = tr_read(tv + to_of(to, mb) + 32 * ss * HD);
        const u32x2 a1 = tr_read(tv + to_of(to, mb) + (32 * ss + 16) * HD);
        const bf16x8 a = as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
#pragma unroll
        for (int qb = 0; qb < NQB; ++qb) acc[mb][qb] = mma16<E>(a, pk[qb], acc[mb][qb]);
      }
      // V^T fragment reads kept four blocks ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        __builtin_amdgcn_sched_group_barrier(0x008, NQB, 0);
        if (mb + 4 < NMB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(0);
    }
    cur = nxt;
  };

  TileCursor cur = first_kv_tile<KT>(P, seg, hk, last);
  if (cur.sp < seg.nspan) issue_kv_tile<kWaves, HD, KT>(wave, lane, cur, s_k0, s_v0);
  while (cur.sp < seg.nspan) {
    step(std::integral_constant<int, 0>{}, cur);
    if (cur.sp >= seg.nspan) break;
    step(std::integral_constant<int, 1>{}, cur);
  }

  // O = acc / l; acc[mb][qb] lane holds d = 16 mb + 4 g4 + i of row qw + 16 qb + j16
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const float ls = rows_sum4(l[qb]);
    const int row = qw + 16 * qb + j16;
    if (row >= T) continue;
    const float inv = ls > 0.f ? 1.f / ls : 0.f;
    bf16* orow = (bf16*)O.ptr + (seg.q_row0 + row) * O.row_stride + (int64_t)h * O.head_stride + 4 * g4;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const f32x4 v = acc[mb][qb] * inv;
      *reinterpret_cast<u32x2*>(orow + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    }
    if (g4 == 0)
      lse[(int64_t)h * lse_ld + seg.q_row0 + row] = ls > 0.f ? (m[qb] + fast_log2(ls)) * kLn2 : neg_inf();
  }
}

// query rows per wave of the forward kernel (32: four waves per work-group; 16: eight)
constexpr int kFwdRowsPerWave = 32;

template <typename E, int HD>
void launch_fwd_generic(const ts_attn_problem& P, int gc, dim3 grid, ts_attn_rows q, ts_attn_rows out, float* lse,
                        int64_t lse_ld, hipStream_t s) {
  ts::TimedLaunch timed_("attention.fwd_kernel", s);
  if constexpr (HD != D) {
    if (gc == 4) {
      hipLaunchKernelGGL((fwd_kernel<E, 4, HD>), grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld);
      return;
    }
  }
  if (gc == 2)
    hipLaunchKernelGGL((fwd_kernel<E, 2, HD>), grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld);
  else
    hipLaunchKernelGGL((fwd_kernel<E, 1, HD>), grid, dim3(kThreads), 0, s, P, q, out, lse, lse_ld);
}

template <typename E>
int launch_fwd_t(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows out, float* lse, int64_t lse_ld,
               hipStream_t s) {
  const int group = P.hq / P.hkv;
  const int gc = heads_per_block(group);
  const dim3 grid((unsigned)(P.n_q_work * P.hkv * (group / gc)));
  switch (P.head_dim) {
    case 32: launch_fwd_generic<E, 32>(P, gc, grid, q, out, lse, lse_ld, s); break;
    case 64: launch_fwd_generic<E, 64>(P, gc, grid, q, out, lse, lse_ld, s); break;
    case 96: launch_fwd_generic<E, 96>(P, gc, grid, q, out, lse, lse_ld, s); break;
    case 192: launch_fwd_generic<E, 192>(P, gc, grid, q, out, lse, lse_ld, s); break;
    case 256: {
      ts::TimedLaunch timed_("attention.fwd_kernel", s);
      if (gc == 4)
        hipLaunchKernelGGL((fwd_wave_kernel<E, 1, 256, 4>), grid, dim3(512), 0, s, P, q, out, lse, lse_ld);
      else if (gc == 2)
        hipLaunchKernelGGL((fwd_wave_kernel<E, 1, 256, 2>), grid, dim3(512), 0, s, P, q, out, lse, lse_ld);
      else
        hipLaunchKernelGGL((fwd_wave_kernel<E, 1, 256, 1>), grid, dim3(512), 0, s, P, q, out, lse, lse_ld);
      break;
    }
    default: {
      ts::TimedLaunch timed_("attention.fwd_kernel", s);
      if (gc == 4)
        hipLaunchKernelGGL((fwd_wave_kernel<E, kFwdRowsPerWave / 16, D, 4, TS_FWD_KT128>), grid,
                           dim3(64 * 128 / kFwdRowsPerWave), 0, s, P, q, out, lse, lse_ld);
      else if (gc == 2)
        hipLaunchKernelGGL((fwd_wave_kernel<E, 2, D, 2, TS_FWD_KT128_GC>), grid, dim3(256), 0, s, P, q, out, lse,
                           lse_ld);
      else
        hipLaunchKernelGGL((fwd_wave_kernel<E, 2, D, 1, TS_FWD_KT128_GC>), grid, dim3(256), 0, s, P, q, out, lse,
                           lse_ld);
    }
  }
  return ts::check_launch("ts_attn_fwd");
}

int launch_fwd(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows out, float* lse, int64_t lse_ld,
               hipStream_t s) {
  return P.dtype == kF16 ? launch_fwd_t<f16>(P, q, out, lse, lse_ld, s) : launch_fwd_t<bf16>(P, q, out, lse, lse_ld, s);
}

}  // namespace attn
}  // namespace ts
