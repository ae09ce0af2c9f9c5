// Attention backward: dK / dV, one wave per query head (GQA groups that are
// a multiple of 4, head dim 128).  A translation unit of its own so that it
// can take its own code-generation flags.
#include "attention_impl.h"

namespace ts {
namespace attn {

// acc += A B on v_mfma_f32_16x16x32_{bf16,f16} with acc held in accumulation
// registers (inline assembly, "a" constraint), while this translation unit,
// compiled with MFMA results in VGPRs, keeps S and dP in VGPRs where the
// softmax arithmetic reads them (no copies out of the accumulation
// registers).  The compiler does not see an MFMA inside the assembly, so the
// hazards it would resolve are resolved here: SETTLE puts the two wait
// states that a VALU write of an A/B operand needs before an MFMA reads it
// in front of the instruction (the first product of each freshly packed
// P / dS operand), and the kernel waits before it reads the accumulators.
template <typename E, bool SETTLE>
__device__ __forceinline__ void mma16_acc(f32x4& acc, bf16x8 a, bf16x8 b) {
  if constexpr (std::is_same_v<E, f16>) {
    if constexpr (SETTLE)
      asm("s_nop 1\n\tv_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    else
      asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  } else {
    if constexpr (SETTLE)
      asm("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    else
      asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  }
}

// a 32-row block of one visit of the work-group's run, with the DMA sources
// of its Q, dO and statistics rows for the wave's current head
struct WaveCursor {
  int vi;           // visit index; >= nvisit at the end
  int r0;           // first row of the block (segment-local)
  int q_len;        // rows of the visited segment
  int off;          // its kv_len - q_len
  int kpos;         // position of the run's first key in the segment's key order
  const bf16* q;    // Q row r0 of the segment, current head
  const bf16* d;    // dO row r0 likewise
  const float* st;  // the row's (lse2, delta) pair
};

// ---------------------------------------------------------------------------
// backward dK / dV, one wave per query head (GQA groups that are a multiple of 4)
//
// A work-group owns 16 KB keys of one run and one KV head; wave w handles query
// heads w, w + 4, ... of the group over all of them, so a wave's LDS reads of
// its head's Q/dO tile feed 16 KB keys of MFMA work.  The K^T and V^T
// operands stay in registers.  Each wave streams its head's 32-row
// Q/dO tiles and their 32 (lse * log2 e, delta) pairs into its own
// double-buffered LDS region with buffer_load ... lds: the buffer resource of
// a tile covers exactly its valid rows, so rows past a segment's end arrive
// as zeros (no clamping, no masking: a zero row has S = dP = 0, statistics
// (0, 0), hence dS = 0 and a zero dO row, and adds nothing), and every
// lane's address is a constant byte offset fixed at kernel start.  Rows are
// 256 bytes, 16-byte chunk c of row r at chunk slot c ^ tile_swizzle(r & 15):
// row reads of 16 rows at one chunk, transpose reads and the DMA's 4-row
// instructions are all conflict-free.  dO^T and Q^T come from ds_read_b64_tr_b16: within each
// 16-lane group, lane i receives column (i & 3) of the rows addressed by
// lanes i/4, i/4 + 4, i/4 + 8, i/4 + 12, so lane j addressing row kbase +
// j/4, columns m0 + 4 (j & 3) yields X[kbase + t][m0 + i], t = 0..3 (pinned
// by the LDS probe test).  The causal mask is applied only to tiles that
// cross the diagonal.  The next block's DMA is issued without a branch
// (zero-size resources past the last block) in the same basic block as the
// score MFMAs, so its scalar set-up interleaves with them, and the visit
// cursor caches its segment's fields, so a step reads no table unless it
// enters the next visit.  The per-head partials are summed across waves
// through LDS in wave order.  On the dS route (DS) a step stores its dS
// blocks right after computing them (the kernel has no registers for a
// deferred copy), through a per-lane pointer that follows the visit cursor.
// ---------------------------------------------------------------------------
template <typename E, int KB, bool DS = false>
__global__ __launch_bounds__(kThreads, 1) void dkdv_wave_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                                ts_attn_rows dO,
                                                                const float* __restrict__ rowstats,
                                                                int64_t lse_ld, DsArgs S) {
  // per wave and stage: Q tile, dO tile, then 32 (lse2, delta) pairs
  __shared__ __attribute__((aligned(16))) bf16 s_b0[4][kStage32];
  __shared__ __attribute__((aligned(16))) bf16 s_b1[4][kStage32];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, j16 = lane & 15;
  int hk;
  const int item = task_of(P.n_kv_work, P.n_kv_long, hk);
  const int run_id = uniform_table(P.kv_work)[2 * item];
  const int k0 = uniform_table(P.kv_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const ts_attn_run run = load_uniform(P.runs, run_id);
  constexpr int NK = 16 * KB;  // keys per work-group
  const int nkeys = min(NK, run.len - k0);
  const float c = P.scale * kLog2e;
  const int nkb = (run.len + 15) >> 4;  // 16-key blocks of the run
  // dS route: this lane's element of key block k0 / 16 in head 0's part;
  // the bookkeeping is kept in VGPRs (derived from an opaque zero), like the
  // key-split kernel's
  int vzero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
  const int64_t ds_head = DS ? S.head + vzero : 0;
  bf16* const ds_base = DS ? (bf16*)S.ptr + (vzero + ds_store_offset(lane) / 2) : nullptr;
  bf16* const ds_lane = ds_base + (int64_t)(k0 >> 4) * kDsBlock;

  // per-lane LDS offsets (elements)
  int ro[4], to[8], dchunk[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ro[ks] = j16 * D + (((4 * ks + g4) ^ tile_swizzle(j16)) << 3);
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int r = 4 * g4 + (j16 >> 2);
    const int col = 16 * mb + 4 * (j16 & 3);
    to[mb] = r * D + ((((col >> 3) ^ tile_swizzle(r)) & 15) << 3) + (col & 7);
  }
  // DMA instruction t fills rows 4t .. 4t + 3; lane (g4, j16) the row 4t + g4,
  // chunk slot j16 with logical chunk j16 ^ tile_swizzle(4 (t & 3) + g4)
#pragma unroll
  for (int t = 0; t < 4; ++t) dchunk[t] = (j16 ^ tile_swizzle(4 * t + g4)) << 3;
  // byte offsets of this lane's row and chunk within a 16-row half tile, less
  // the 1024 t that DMA instruction t adds to both addresses as its
  // instruction offset (a row stride is at least 128 elements, so they stay
  // non-negative)
  int qoff[4], doff[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    qoff[t] = (int)(((4 * t + g4) * Q.row_stride + dchunk[t]) * 2) - 1024 * t;
    doff[t] = (int)(((4 * t + g4) * dO.row_stride + dchunk[t]) * 2) - 1024 * t;
  }
  const int64_t q32 = 32 * Q.row_stride, d32 = 32 * dO.row_stride;  // one block of rows
  const int64_t q16 = 16 * Q.row_stride, d16 = 16 * dO.row_stride;  // its upper half
  const uint32_t qrow_bytes = (uint32_t)(Q.row_stride * 2), drow_bytes = (uint32_t)(dO.row_stride * 2);

  // K^T and V^T operands: kreg[kb][ks] = K[k0 + 16 kb + j16][32 ks + 8 g4 ..], vreg likewise
  bf16x8 kreg[KB][4], vreg[KB][4];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = 16 * kb + j16;
    const bf16* kp = (const bf16*)run.k + (int64_t)(k0 + key) * run.k_row_stride + (int64_t)hk * run.k_head_stride;
    const bf16* vp = (const bf16*)run.v + (int64_t)(k0 + key) * run.v_row_stride + (int64_t)hk * run.v_head_stride;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kreg[kb][ks] = as_bf16x8(key < nkeys ? ld16(kp + 32 * ks + 8 * g4) : u32x4{0u, 0u, 0u, 0u});
      vreg[kb][ks] = as_bf16x8(key < nkeys ? ld16(vp + 32 * ks + 8 * g4) : u32x4{0u, 0u, 0u, 0u});
    }
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

  int hh = 0;  // the wave's current head
  // enter visit c.vi (< nvisit): cache its segment's fields and start at the
  // first 32-row block whose rows can see key k0, with that block's Q, dO and
  // statistics rows of head hh
  auto enter = [&](WaveCursor& c) {
    const ts_attn_ref ref = load_uniform(P.run_visits, run.visit0 + c.vi);
    const ts_attn_segment seg = load_uniform(P.segs, ref.index);
    c.q_len = seg.q_len;
    c.off = seg.kv_len - seg.q_len;
    c.kpos = ref.kpos;
    const int rs = ref.kpos + k0 - c.off;
    c.r0 = (rs < 0 ? 0 : rs) & ~31;
    const int64_t row0 = seg.q_row0 + c.r0;
    c.q = (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)hh * Q.head_stride;
    c.d = (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)hh * dO.head_stride;
    c.st = rowstats + 2 * ((int64_t)hh * lse_ld + row0);
  };
  // first block at or after c; skips visits with no visible rows
  auto settle = [&](WaveCursor c) -> WaveCursor {
    while (c.r0 >= c.q_len) {
      if (++c.vi >= run.nvisit) break;
      enter(c);
    }
    return c;
  };
  auto first = [&]() -> WaveCursor {
    WaveCursor c{0, 0, 0, 0, 0, nullptr, nullptr, nullptr};
    if (run.nvisit > 0) enter(c);
    return settle(c);
  };
  // dS route: this lane's element of block k0 / 16 of c's row block in head
  // hh's part (c on a visit)
  auto locate = [&](const WaveCursor& c) -> bf16* {
    // consumed here, so that no scalar load is outstanding when the next
    // step's LDS reads count their completions
    const int64_t blk = load_uniform(S.visit, run.visit0 + c.vi) / kDsBlock +
                        ds_blocks_before(DsRect{c.off - c.kpos, nkb, c.q_len}, c.r0 >> 5);
    asm volatile("" ::"s"(blk));
    return ds_lane + (int64_t)hh * ds_head + blk * kDsBlock;
  };
  // the block after c (settled: past its visit's rows, the next visit's
  // first): within a visit the DMA sources advance by 32 rows; dS route:
  // `at` follows it, advanced by c's row block's block count within a visit,
  // located afresh on entering the next
  auto next_block = [&](WaveCursor c, bf16*& at) -> WaveCursor {
    int inc = 0;
    if constexpr (DS) {
      const int last = c.off - c.kpos + min(c.r0 + 31, c.q_len - 1);
      inc = last < 0 ? 0 : min(nkb, (last >> 4) + 1);
    }
    const int vi0 = c.vi;
    c.r0 += 32;
    c.q += q32;
    c.d += d32;
    c.st += 64;
    if (c.r0 >= c.q_len) c = settle(c);  // tables are read only here
    if constexpr (DS) {
      if (c.vi == vi0)
        at += (int64_t)inc * kDsBlock;
      else if (c.vi < run.nvisit)
        at = locate(c);
    }
    return c;
  };
  // DMA of block `cur` (nothing, as zero-size buffer resources, when it is
  // past the run's last visit): each of the four 4 KB quarters of the Q and
  // dO tiles is four instructions under one M0, instruction t at instruction
  // offset 1024 t
  auto issue = [&](const WaveCursor& cur, bf16* buf) {
    const int nrows = max(0, min(32, cur.q_len - cur.r0));
    const int n_lo = min(16, nrows), n_hi = nrows - n_lo;
    const rsrc_t q_lo = make_rsrc(cur.q, n_lo * qrow_bytes);
    const rsrc_t q_hi = make_rsrc(cur.q + q16, n_hi * qrow_bytes);
    const rsrc_t d_lo = make_rsrc(cur.d, n_lo * drow_bytes);
    const rsrc_t d_hi = make_rsrc(cur.d + d16, n_hi * drow_bytes);
    auto quarter = [&](const rsrc_t& r, bf16* lds, const int (&voff)[4]) __attribute__((always_inline)) {
      buffer_dma16_at<0>(r, lds, voff[0]);
      buffer_dma16_at<1024>(r, lds, voff[1]);
      buffer_dma16_at<2048>(r, lds, voff[2]);
      buffer_dma16_at<3072>(r, lds, voff[3]);
    };
    quarter(q_lo, buf, qoff);
    quarter(q_hi, buf + 4 * 512, qoff);
    quarter(d_lo, buf + kTile32, doff);
    quarter(d_hi, buf + kTile32 + 4 * 512, doff);
    // 32 rows x 8 bytes of statistics: lanes 0..15, 16 bytes each (the other
    // lanes read past the resource and write zeros after them)
    const rsrc_t rs = make_rsrc(cur.st, (uint32_t)(nrows * 8));
    buffer_dma16(rs, buf + 2 * kTile32, lane < 16 ? lane * 16 : 0x7ffffff0);
  };

  // one 32-row block of the current head; buffer roles fixed per call
  // `nxt` is the block after `cur`, already settled: the step's body up to the
  // cursor update is branch-free, so the next block's DMA set-up interleaves
  // with the MFMAs
  auto step = [&](auto bsel, WaveCursor& cur, WaveCursor& nxt, bf16*& cur_at, bf16*& nxt_at) {
      const int off = cur.off, r0 = cur.r0, kpos = cur.kpos;
      __builtin_amdgcn_s_waitcnt(0);  // this block's tiles have landed
      // static buffer roles: the LDS reads below and the prefetch into the other
      // buffer touch different arrays, so no wait for the prefetch is needed
      bf16* cur_buf = bsel.value == 0 ? s_b0[wave] : s_b1[wave];
      bf16* nxt_buf = bsel.value == 0 ? s_b1[wave] : s_b0[wave];
      issue(nxt, nxt_buf);
      const bf16* tq = cur_buf;
      const bf16* td = cur_buf + kTile32;
      const float* sl = reinterpret_cast<const float*>(cur_buf + 2 * kTile32);  // [32] (lse2, delta)

      // S = Q K^T, dP - delta = dO V^T - delta (the dP accumulators start at
      // -delta of their rows, so that dS = P (dP - delta) is one multiply):
      // [qb][kb] holds rows 16 qb + 4 g4 + i, key 16 kb + j16
      f32x4 ndl[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) ndl[qb][i] = -sl[2 * (16 * qb + 4 * g4 + i) + 1];
      f32x4 sc[2][KB], dp[2][KB];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          sc[qb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[qb][kb] = ndl[qb];
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
  #pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            sc[qb][kb] = mma16<E>(aq[qb], kreg[kb][ks], sc[qb][kb]);
            dp[qb][kb] = mma16<E>(ad[qb], vreg[kb][ks], dp[qb][kb]);
          }
        }
      }
      // Q/dO row reads two k-steps ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        __builtin_amdgcn_sched_group_barrier(0x008, 4 * KB, 0);
        if (ks + 2 < 4) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      }
      // this lane's rows: 16 qb + 4 g4 + i
      float l2[2][4];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) l2[qb][i] = sl[2 * (16 * qb + 4 * g4 + i)];
      // P and dS as B operands: slot j = 4 qb + i  <->  row 16 qb + 4 g4 + i
      bf16x8 pk[KB], dsk[KB];
      // the block crosses the diagonal (or, when dS is stored, the run's end:
      // P of a key past it, whose K row is zero, is exp2(-lse2), not 0)
      if ((kpos + k0 + NK - 1 > off + r0) | (DS && nkeys < NK)) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          // row rl sees the key iff rl >= -lim; dS route: a key past the run
          // is put past every row (2^24 rows)
          const int lim = off + r0 - kpos - (k0 + 16 * kb + j16) - (DS && 16 * kb + j16 >= nkeys ? (1 << 24) : 0);
          float pv[8], dsv[8];
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int rl = 16 * qb + 4 * g4 + i;
              const float p = rl + lim >= 0 ? fast_exp2(sc[qb][kb][i] * c - l2[qb][i]) : 0.f;
              pv[4 * qb + i] = p;
              dsv[4 * qb + i] = p * dp[qb][kb][i];
            }
          pk[kb] = pack8<E>(pv);
          dsk[kb] = pack8<E>(dsv);
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
              dsv[4 * qb + i] = p * dp[qb][kb][i];
            }
          pk[kb] = pack8<E>(pv);
          dsk[kb] = pack8<E>(dsv);
        }
      }
      if constexpr (DS) {
        // this step's dS blocks (key blocks k0 / 16 + kb of row block r0 / 32)
        // that the rectangle holds
        const int last = off - kpos + min(r0 + 31, cur.q_len - 1);
        const int nb = (last < 0 ? 0 : min(nkb, (last >> 4) + 1)) - (k0 >> 4);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
          if (kb < nb) global_st16(cur_at + kb * kDsBlock, as_u32x4(dsk[kb]));
      }
      // dV^T += dO^T P, dK^T += Q^T dS: rows d = 16 mb + 4 g4 + i, column key;
      // the dO^T / Q^T fragments of block mb + 2 are read while block mb's
      // MFMAs run
      bf16x8 a_do[3], a_q[3];
      auto frag = [&](int mb, bf16x8& fd, bf16x8& fq) __attribute__((always_inline)) {
        const u32x2 a0 = tr_read(td + to[mb]), a1 = tr_read(td + to[mb] + 16 * D);
        const u32x2 b0 = tr_read(tq + to[mb]), b1 = tr_read(tq + to[mb] + 16 * D);
        fd = as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
        fq = as_bf16x8(u32x4{b0[0], b0[1], b1[0], b1[1]});
      };
      frag(0, a_do[0], a_q[0]);
      frag(1, a_do[1], a_q[1]);
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        if (mb + 2 < 8) frag(mb + 2, a_do[(mb + 2) % 3], a_q[(mb + 2) % 3]);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          if (mb == 0) {
            mma16_acc<E, true>(dv[mb][kb], a_do[mb % 3], pk[kb]);
            mma16_acc<E, true>(dk[mb][kb], a_q[mb % 3], dsk[kb]);
          } else {
            mma16_acc<E, false>(dv[mb][kb], a_do[mb % 3], pk[kb]);
            mma16_acc<E, false>(dk[mb][kb], a_q[mb % 3], dsk[kb]);
          }
        }
      }
      // keep the reads two blocks ahead (the scheduler otherwise pulls them
      // back to one block ahead, where six MFMAs do not cover their latency)
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * KB, 0);
        if (mb + 2 < 8) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      }
      cur = nxt;
      if constexpr (DS) cur_at = nxt_at;
      nxt = next_block(nxt, nxt_at);
  };

  for (int g = wave; g < group; g += 4) {
    hh = hk * group + g;
    WaveCursor cur = first();
    bf16* cur_at = ds_lane;
    if constexpr (DS)
      if (cur.vi < run.nvisit) cur_at = locate(cur);
    bf16* nxt_at = cur_at;
    WaveCursor nxt = next_block(cur, nxt_at);
    __builtin_amdgcn_s_waitcnt(0);  // the previous head's last (empty) DMA has landed
    if (cur.vi < run.nvisit) issue(cur, s_b0[wave]);
    while (cur.vi < run.nvisit) {
      step(std::integral_constant<int, 0>{}, cur, nxt, cur_at, nxt_at);
      if (cur.vi >= run.nvisit) break;
      step(std::integral_constant<int, 1>{}, cur, nxt, cur_at, nxt_at);
    }
  }

  // sum the waves' partials in wave order: wave w stages [NK keys][128 d] fp32
  // (16-byte chunk c of key k at slot c ^ (k & 31)) in s_b0[2w] (w < 2) or
  // s_b1[2(w - 2)], 2 x kStage32 bf16 >= 32 KB; every thread then adds the
  // four partials of its outputs
  // the wait states between the last MFMA writing the accumulators and the
  // first reads of them (the compiler does not see those MFMAs)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
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
        st16((bf16*)base + (int64_t)(k0 + key) * rs + (int64_t)hk * hs + d8, as_u32x4(pack8<E>(acc8)));
    }
    __syncthreads();
  }
}

template <typename E, bool DS>
void launch_dkdv_wave(dim3 grid, const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout,
                      const float* rowstats, int64_t lse_ld, const DsArgs& S, hipStream_t s) {
  hipLaunchKernelGGL((dkdv_wave_kernel<E, 3, DS>), grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, S);
}

template void launch_dkdv_wave<bf16, false>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows,
                                            const float*, int64_t, const DsArgs&, hipStream_t);
template void launch_dkdv_wave<bf16, true>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows,
                                           const float*, int64_t, const DsArgs&, hipStream_t);
template void launch_dkdv_wave<f16, false>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows,
                                           const float*, int64_t, const DsArgs&, hipStream_t);
template void launch_dkdv_wave<f16, true>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows,
                                          const float*, int64_t, const DsArgs&, hipStream_t);

}  // namespace attn
}  // namespace ts
