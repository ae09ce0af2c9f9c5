// Attention backward: dK / dV at head dim 256 with 32 keys per wave (every
// GQA group: at this head dim the work items hold 64 keys).  A
// translation unit of its own so that it can take its own code-generation
// flags (MFMA results in VGPRs, the dK/dV accumulators in accumulation
// registers through inline assembly).
#include "attention_impl.h"

namespace ts {
namespace attn {

namespace {

// acc += A B on v_mfma_f32_16x16x32_{bf16,f16} with acc in accumulation
// registers (inline assembly, "a" constraint).  The compiler does not see the
// MFMA inside the assembly, so the hazards it would resolve are resolved
// here: SETTLE puts the two wait states that a VALU write of an A/B operand
// needs in front of the instruction (the first product of each freshly packed
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

}  // namespace

// ---------------------------------------------------------------------------
// backward dK / dV at head dim 256, two waves of 32 keys per work-group
//
// A work-group owns the work item's 64 keys of one run and one KV head; wave
// w owns keys 32 w .. 32 w + 31 as two 16-key blocks (kb), their K^T and V^T
// in registers (128 VGPRs) and their dK^T / dV^T accumulators in the 256
// accumulation registers.  Both waves walk the same steps -- every query head
// of the group, then every visible 32-row block -- over one double-buffered
// LDS stage that they fill together by buffer DMA (the Q and dO rows of the
// step, 16-byte chunk c of row r at slot c ^ tile_swizzle(r & 15), and the
// rows' 32 (lse * log2 e, delta) pairs), one work-group barrier per step; two
// work-groups share a CU (one wave per SIMD).  A Q/dO row fragment read from
// LDS feeds the MFMAs of both key blocks, so the LDS reads per MFMA are half
// those of the 16-keys-per-wave kernel, whose four waves each read the whole
// stage for one block.  The buffer resource of a half tile covers exactly its
// valid rows: rows past a segment's end arrive as zeros and add nothing (S =
// dP = 0, statistics (0, 0)).  S = Q K^T and dP = dO V^T take the Q/dO rows as
// A operands; dV^T += dO^T P and dK^T += Q^T dS take dO^T / Q^T from
// ds_read_b64_tr_b16 (the lane layouts of the other dK/dV kernels).  Only
// key blocks that cross the diagonal (or, when dS is stored, the run's end)
// are masked.  On the dS route the dS blocks of a step that the rectangle
// holds are stored by the next step, right after it issues its DMA (a store
// issued before the dV/dK products held them up in the memory queue: 4.31
// against 4.10 ms on the branch shape).
// ---------------------------------------------------------------------------
template <typename E, bool DS>
__global__ __launch_bounds__(128, 1) void dkdv256_kernel(ts_attn_problem P, ts_attn_rows Q, ts_attn_rows dO,
                                                        const float* __restrict__ rowstats, int64_t lse_ld,
                                                        DsArgs S) {
  constexpr int HD = 256;
  constexpr int NKS = HD / 32;           // k-steps of S / dP over the head dim
  constexpr int NMB = HD / 16;           // 16-column blocks of dK / dV
  constexpr int KB = 2;                  // 16-key blocks per wave
  constexpr int TILE = 32 * HD;          // elements of a 32-row tile
  constexpr int STAGE = 2 * TILE + 512;  // Q, dO, then 1 KB of statistics
  constexpr int RA = 1;                  // k-steps the Q/dO row reads run ahead of their MFMAs
  constexpr int TRA = 2;                 // blocks the dO^T / Q^T reads run ahead of theirs
  __shared__ __attribute__((aligned(16))) bf16 s_b0[STAGE];
  __shared__ __attribute__((aligned(16))) bf16 s_b1[STAGE];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g4 = lane >> 4, j16 = lane & 15;
  int hk;
  const int item = task_of(P.n_kv_work, P.n_kv_long, hk);
  const int run_id = uniform_table(P.kv_work)[2 * item];
  const int k0 = uniform_table(P.kv_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const ts_attn_run run = load_uniform(P.runs, run_id);
  const int wk0 = k0 + 32 * wave;  // the wave's first key (run-local)
  const bool wave_active = wk0 < run.len;  // wave-uniform
  const float c = P.scale * kLog2e;
  const int nkb = (run.len + 15) >> 4;  // 16-key blocks of the run

  int ro[4], to[8];
  swizzled_offsets<HD>(lane, ro, to);
  // DMA: a tile is 16 instructions of two rows (lane l: row 2 t + l / 32, slot
  // l % 32 with logical chunk (l % 32) ^ tile_swizzle(row & 15)); wave w issues
  // t = w + 2 u.  The instructions of rows 16 .. 31 (u = 4 .. 7) take the
  // upper half tile's resource, 16 rows on, with the byte offsets of u - 4.
  int qoff[4], doff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = 2 * (wave + 2 * u) + (lane >> 5);
    const int chunk = (lane & 31) ^ tile_swizzle(row & 15);
    qoff[u] = (int)((row * Q.row_stride + chunk * 8) * 2);
    doff[u] = (int)((row * dO.row_stride + chunk * 8) * 2);
  }

  // K^T and V^T operands: kreg[kb][ks] = K[key wk0 + 16 kb + j16][32 ks + 8 g4 ..], vreg likewise
  bf16x8 kreg[KB][NKS], vreg[KB][NKS];
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = wk0 + 16 * kb + j16;
    const bool valid = key < run.len;
    const bf16* kp = (const bf16*)run.k + (int64_t)key * run.k_row_stride + (int64_t)hk * run.k_head_stride;
    const bf16* vp = (const bf16*)run.v + (int64_t)key * run.v_row_stride + (int64_t)hk * run.v_head_stride;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      kreg[kb][ks] = as_bf16x8(valid ? ld16(kp + 32 * ks + 8 * g4) : u32x4{0u, 0u, 0u, 0u});
      vreg[kb][ks] = as_bf16x8(valid ? ld16(vp + 32 * ks + 8 * g4) : u32x4{0u, 0u, 0u, 0u});
    }
  }
  f32x4 dk[NMB][KB], dv[NMB][KB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb)
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      dk[mb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
      dv[mb][kb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  // dS route: this lane's element of key block wk0 / 16 (head 0's part); the
  // bookkeeping is kept in VGPRs (derived from an opaque zero), as in the
  // other dK/dV kernels
  int vzero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
  const int64_t ds_head = DS ? S.head + vzero : 0;
  bf16* const ds_base = DS ? (bf16*)S.ptr + (vzero + ds_store_offset(lane) / 2) : nullptr;
  bf16* const ds_lane = ds_base + (int64_t)(wk0 >> 4) * kDsBlock;
  // step cursor: query head g of the group, then the visit / row block
  struct Cursor {
    int g;
    VisitCursor v;
    bf16* at;  // dS route: this lane's element of the step's first dS block
  };
  auto enter = [&](VisitCursor& cv) {
    const ts_attn_ref ref = load_uniform(P.run_visits, run.visit0 + cv.vi);
    const ts_attn_segment seg = load_uniform(P.segs, ref.index);
    cv.q_len = seg.q_len;
    cv.off = seg.kv_len - seg.q_len;
    cv.kpos = ref.kpos;
    cv.q_row0 = seg.q_row0;
    const int rs = ref.kpos + k0 - cv.off;
    cv.r0 = (rs < 0 ? 0 : rs) & ~31;
  };
  auto settle = [&](VisitCursor cv) -> VisitCursor {
    while (cv.r0 >= cv.q_len) {
      if (++cv.vi >= run.nvisit) break;
      enter(cv);
    }
    return cv;
  };
  auto first_visit = [&]() -> VisitCursor {
    VisitCursor cv{0, 0, 0, 0, 0, 0};
    if (run.nvisit > 0) enter(cv);
    return settle(cv);
  };
  // `at` of a cursor on a visit (its rectangle's offset, the blocks of the
  // row blocks before r0 / 32)
  auto locate = [&](const Cursor& cu) -> bf16* {
    const int64_t blk = load_uniform(S.visit, run.visit0 + cu.v.vi) / kDsBlock +
                        ds_blocks_before(DsRect{cu.v.off - cu.v.kpos, nkb, cu.v.q_len}, cu.v.r0 >> 5);
    asm volatile("" ::"s"(blk));
    return ds_lane + (int64_t)(hk * group + cu.g) * ds_head + blk * kDsBlock;
  };
  // the step after `cu`; g == group at the end
  auto advance = [&](Cursor cu) -> Cursor {
    int inc = 0;  // dS route: blocks of the row block being left
    if constexpr (DS) {
      const int last = cu.v.off - cu.v.kpos + min(cu.v.r0 + 31, cu.v.q_len - 1);
      inc = last < 0 ? 0 : min(nkb, (last >> 4) + 1);
    }
    bool next_row_block = true;  // same visit and head
    cu.v.r0 += 32;
    if (cu.v.r0 >= cu.v.q_len) {
      cu.v = settle(cu.v);
      next_row_block = false;
    }
    if (cu.v.vi >= run.nvisit) {
      ++cu.g;
      cu.v = first_visit();
      next_row_block = false;
    }
    if constexpr (DS) {
      if (next_row_block)
        cu.at += (int64_t)inc * kDsBlock;
      else if (cu.g < group && cu.v.vi < run.nvisit)
        cu.at = locate(cu);
    }
    return cu;
  };
  // DMA of step `cu`'s tiles into `buf` (zero-size resources when cu is past
  // the end, so the instructions need no branch)
  auto issue = [&](const Cursor& cu, bf16* buf) {
    const bool live = cu.g < group && cu.v.vi < run.nvisit;
    const int nrows = live ? max(0, min(32, cu.v.q_len - cu.v.r0)) : 0;
    const int n_lo = min(16, nrows), n_hi = nrows - n_lo;
    const int h = hk * group + (live ? cu.g : 0);
    const int64_t row0 = live ? cu.v.q_row0 + cu.v.r0 : 0;
    const bf16* qb = (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)h * Q.head_stride;
    const bf16* db = (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)h * dO.head_stride;
    const rsrc_t q_lo = make_rsrc(qb, (uint32_t)(n_lo * Q.row_stride * 2));
    const rsrc_t q_hi = make_rsrc(qb + 16 * Q.row_stride, (uint32_t)(n_hi * Q.row_stride * 2));
    const rsrc_t d_lo = make_rsrc(db, (uint32_t)(n_lo * dO.row_stride * 2));
    const rsrc_t d_hi = make_rsrc(db + 16 * dO.row_stride, (uint32_t)(n_hi * dO.row_stride * 2));
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = wave + 2 * u;
      buffer_dma16(q_lo, buf + t * 512, qoff[u]);
      buffer_dma16(q_hi, buf + (t + 8) * 512, qoff[u]);
      buffer_dma16(d_lo, buf + TILE + t * 512, doff[u]);
      buffer_dma16(d_hi, buf + TILE + (t + 8) * 512, doff[u]);
    }
    if (wave == 0) {
      // 32 rows x 8 bytes of statistics: lanes 0..15, 16 bytes each (the
      // other lanes read past the resource and write zeros after them)
      const rsrc_t rs = make_rsrc(rowstats + 2 * ((int64_t)h * lse_ld + row0), (uint32_t)(nrows * 8));
      buffer_dma16(rs, buf + 2 * TILE, lane < 16 ? lane * 16 : 0x7ffffff0);
    }
  };

  // dS route: the previous step's dS blocks, stored after the next DMA issue
  bf16x8 pend[KB];
  bf16* pend_at = ds_lane;
  int pend_nb = 0;
  // one step on the tiles in `cur_buf`; buffer roles fixed per call
  auto step = [&](auto bsel, Cursor& cur, Cursor& nxt) {
    bf16* cur_buf = bsel.value == 0 ? s_b0 : s_b1;
    bf16* nxt_buf = bsel.value == 0 ? s_b1 : s_b0;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the step's tiles has landed
    __syncthreads();                // the other wave's has, and nobody reads nxt_buf any more
    issue(nxt, nxt_buf);
    if constexpr (DS) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
        if (kb < pend_nb) global_st16(pend_at + kb * kDsBlock, as_u32x4(pend[kb]));
      pend_nb = 0;
    }
    const int off = cur.v.off, r0 = cur.v.r0, kpos = cur.v.kpos;
    const int nrows = min(32, cur.v.q_len - r0);
    // the wave's keys are all invisible to this block when its first key is
    // beyond the block's last row
    const bool live = wave_active && kpos + wk0 <= off + r0 + nrows - 1;
    if (live) {
      const bf16* tq = cur_buf;
      const bf16* td = cur_buf + TILE;
      const float* sl = reinterpret_cast<const float*>(cur_buf + 2 * TILE);  // [32] (lse2, delta)
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
      for (int ks = 0; ks < NKS; ++ks) {
        bf16x8 aq[2], ad[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          aq[qb] = as_bf16x8(ld16(tq + ro_of(ro, ks) + 16 * qb * HD));
          ad[qb] = as_bf16x8(ld16(td + ro_of(ro, ks) + 16 * qb * HD));
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb) {
            sc[qb][kb] = mma16<E>(aq[qb], kreg[kb][ks], sc[qb][kb]);
            dp[qb][kb] = mma16<E>(ad[qb], vreg[kb][ks], dp[qb][kb]);
          }
      }
      // Q/dO row reads RA k-steps ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 4 * RA, 0);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        __builtin_amdgcn_sched_group_barrier(0x008, 4 * KB, 0);
        if (ks + RA < NKS) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
      // P and dS as B operands: slot j = 4 qb + i  <->  row 16 qb + 4 g4 + i
      bf16x8 pk[KB], dsk[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        // row rl sees key wk0 + 16 kb + j16 iff rl >= -lim; dS route: a key past
        // the run is put past every row (2^24 rows), so that its P is zero too
        // (its K row is zero, so exp2(-lse2) otherwise)
        const int key = wk0 + 16 * kb + j16;
        const int lim = off + r0 - kpos - key - (DS && key >= run.len ? (1 << 24) : 0);
        // wave-uniform: the block crosses the diagonal or the run's end
        const bool diag = (kpos + wk0 + 16 * kb + 15 > off + r0) | (DS && wk0 + 16 * kb + 16 > run.len);
        float pv[8], dsv[8];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rl = 16 * qb + 4 * g4 + i;
            float p = fast_exp2(sc[qb][kb][i] * c - sl[2 * rl]);
            if (diag && rl + lim < 0) p = 0.f;
            pv[4 * qb + i] = p;
            dsv[4 * qb + i] = p * (dp[qb][kb][i] - sl[2 * rl + 1]);
          }
        pk[kb] = pack8<E>(pv);
        dsk[kb] = pack8<E>(dsv);
      }
      if constexpr (DS) {
        // this step's dS blocks (key blocks wk0 / 16 + kb of row block r0 / 32)
        // that the rectangle holds
        const int last = off - kpos + min(r0 + 31, cur.v.q_len - 1);
        const int nb = (last < 0 ? 0 : min(nkb, (last >> 4) + 1)) - (wk0 >> 4);
        pend_nb = nb;
        pend_at = cur.at;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) pend[kb] = dsk[kb];
      }
      __builtin_amdgcn_sched_barrier(0);
      // dV^T += dO^T P, dK^T += Q^T dS: rows d = 16 mb + 4 g4 + i, column key 16 kb + j16
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const int o = to_of(to, mb);
        const u32x2 a0 = tr_read(td + o), a1 = tr_read(td + o + 16 * HD);
        const u32x2 b0 = tr_read(tq + o), b1 = tr_read(tq + o + 16 * HD);
        const bf16x8 a = as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
        const bf16x8 b = as_bf16x8(u32x4{b0[0], b0[1], b1[0], b1[1]});
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          if (mb == 0) {
            mma16_acc<E, true>(dv[mb][kb], a, pk[kb]);
            mma16_acc<E, true>(dk[mb][kb], b, dsk[kb]);
          } else {
            mma16_acc<E, false>(dv[mb][kb], a, pk[kb]);
            mma16_acc<E, false>(dk[mb][kb], b, dsk[kb]);
          }
        }
      }
      // the dO^T / Q^T reads TRA blocks ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 4 * TRA, 1);
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2 * KB, 1);
        if (mb + TRA < NMB) __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
      }
    }
    cur = nxt;
    nxt = advance(nxt);
  };

  Cursor cur{0, first_visit(), ds_lane};
  if (cur.v.vi >= run.nvisit) cur.g = group;  // a run nobody reads
  if constexpr (DS)
    if (cur.g < group) cur.at = locate(cur);
  Cursor nxt = cur.g < group ? advance(cur) : cur;
  issue(cur, s_b0);
  while (cur.g < group) {
    step(std::integral_constant<int, 0>{}, cur, nxt);
    if (cur.g >= group) break;
    step(std::integral_constant<int, 1>{}, cur, nxt);
  }
  if constexpr (DS) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
      if (kb < pend_nb) global_st16(pend_at + kb * kDsBlock, as_u32x4(pend[kb]));
  }
  __builtin_amdgcn_s_waitcnt(0);  // the last (empty) DMA has landed before the waves exit
  // the wait states between the last MFMA writing the accumulators and the
  // first reads of them (the compiler does not see those MFMAs)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  // lane (g4, j16) holds d = 16 mb + 4 g4 .. + 3 of key wk0 + 16 kb + j16: 8-byte stores
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const int key = wk0 + 16 * kb + j16;
    if (key >= run.len) continue;
    if (run.dk) {
      bf16* p = (bf16*)run.dk + (int64_t)key * run.dk_row_stride + (int64_t)hk * run.dk_head_stride + 4 * g4;
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const f32x4 v = dk[mb][kb] * P.scale;
        *reinterpret_cast<u32x2*>(p + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
      }
    }
    if (run.dv) {
      bf16* p = (bf16*)run.dv + (int64_t)key * run.dv_row_stride + (int64_t)hk * run.dv_head_stride + 4 * g4;
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const f32x4 v = dv[mb][kb];
        *reinterpret_cast<u32x2*>(p + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
      }
    }
  }
}

template <typename E, bool DS>
void launch_dkdv256(dim3 grid, const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout, const float* rowstats,
                    int64_t lse_ld, const DsArgs& S, hipStream_t s) {
  hipLaunchKernelGGL((dkdv256_kernel<E, DS>), grid, dim3(128), 0, s, P, q, dout, rowstats, lse_ld, S);
}

template void launch_dkdv256<bf16, false>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows, const float*,
                                          int64_t, const DsArgs&, hipStream_t);
template void launch_dkdv256<bf16, true>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows, const float*,
                                         int64_t, const DsArgs&, hipStream_t);
template void launch_dkdv256<f16, false>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows, const float*,
                                         int64_t, const DsArgs&, hipStream_t);
template void launch_dkdv256<f16, true>(dim3, const ts_attn_problem&, ts_attn_rows, ts_attn_rows, const float*,
                                        int64_t, const DsArgs&, hipStream_t);

}  // namespace attn
}  // namespace ts
