// Attention backward: dK / dV (key-stationary, deterministic).
#include "attention_impl.h"

namespace ts {
namespace attn {

// ---------------------------------------------------------------------------
// backward dK / dV (key-stationary)
// ---------------------------------------------------------------------------
// Register-staged dK/dV for any supported head dim HD and GQA groups that are
// not a multiple of 4 (and, at head dims other than 128, those that are): a
// work-group owns P.kv_block keys (48 or 64) of one run and one KV head, wave
// w keys 16 w .. 16 w + 15 (a wave past the block only helps stage the
// tiles), and loops over every query head of the group and every visible
// 32-row block; Q and dO rows pass through registers into padded LDS rows,
// dO^T and Q^T come from ds_read_b64_tr_b16 (tr_frag).
template <typename E, int HD>
__global__ __launch_bounds__(kThreads, HD > 128 ? 1 : 2) void dkdv_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                           ts_attn_rows dO, const float* __restrict__ rowstats,
                                                           int64_t lse_ld) {
  constexpr int NMB = HD / 16;  // 16-column blocks of dK / dV
  __shared__ __attribute__((aligned(16))) bf16 sq[32 * pitch_of<HD>()];
  __shared__ __attribute__((aligned(16))) bf16 sd[32 * pitch_of<HD>()];
  __shared__ float s_lse2[32];
  __shared__ float s_dlt[32];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int hk;
  const int item = task_of(P.n_kv_work, P.n_kv_long, hk);
  const int run_id = uniform_table(P.kv_work)[2 * item];
  const int k0 = uniform_table(P.kv_work)[2 * item + 1];
  const int group = P.hq / P.hkv;
  const ts_attn_run run = load_uniform(P.runs, run_id);
  const int wk0 = k0 + 16 * wave;                 // first key (run-local) of this wave
  const int mykey = wk0 + (lane & 15);            // key column this lane holds
  const bool in_block = 16 * wave < P.kv_block;   // the wave's keys belong to this work item
  const bool wave_has_keys = in_block && wk0 < run.len;
  const bool key_valid = in_block && mykey < run.len;
  const float c = P.scale * kLog2e;

  // K^T / V^T B operands: key (lane & 15), d = 32 ks + 8 (lane >> 4) .. +7
  bf16x8 kreg[HD / 32], vreg[HD / 32];
  {
    const bf16* kp = (const bf16*)run.k + (int64_t)mykey * run.k_row_stride + (int64_t)hk * run.k_head_stride;
    const bf16* vp = (const bf16*)run.v + (int64_t)mykey * run.v_row_stride + (int64_t)hk * run.v_head_stride;
#pragma unroll
    for (int ks = 0; ks < HD / 32; ++ks) {
      u32x4 a = u32x4{0u, 0u, 0u, 0u}, b = u32x4{0u, 0u, 0u, 0u};
      if (key_valid) {
        a = ld16(kp + 32 * ks + 8 * (lane >> 4));
        b = ld16(vp + 32 * ks + 8 * (lane >> 4));
      }
      kreg[ks] = as_bf16x8(a);
      vreg[ks] = as_bf16x8(b);
    }
  }
  f32x4 dk[NMB], dv[NMB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
    dk[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
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
        rows32_to_lds<HD>(sq, (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)h * Q.head_stride,
                          Q.row_stride, nrows, tid);
        rows32_to_lds<HD>(sd, (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)h * dO.head_stride,
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
          for (int ks = 0; ks < HD / 32; ++ks) {
            const int r = 16 * qb + (lane & 15);
            const bf16x8 aq = as_bf16x8(ld16(sq + r * pitch_of<HD>() + 32 * ks + 8 * (lane >> 4)));
            const bf16x8 ad = as_bf16x8(ld16(sd + r * pitch_of<HD>() + 32 * ks + 8 * (lane >> 4)));
            s[qb] = mma16<E>(aq, kreg[ks], s[qb]);
            dp[qb] = mma16<E>(ad, vreg[ks], dp[qb]);
          }
        }
        float pv[8], dsv[8];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rl = 16 * qb + 4 * (lane >> 4) + i;
            float p = fast_exp2(s[qb][i] * c - s_lse2[rl]);
            if (rl >= nrows || !key_valid || ref.kpos + mykey > off + r0 + rl) p = 0.f;
            pv[4 * qb + i] = p;
            dsv[4 * qb + i] = p * (dp[qb][i] - s_dlt[rl]);
          }
        const bf16x8 pk = pack8<E>(pv);
        const bf16x8 dsk = pack8<E>(dsv);
#pragma unroll
        for (int mb = 0; mb < NMB; ++mb) {
          dv[mb] = mma16<E>(tr_frag<HD>(sd, 0, mb, lane), pk, dv[mb]);
          dk[mb] = mma16<E>(tr_frag<HD>(sq, 0, mb, lane), dsk, dk[mb]);
        }
      }
    }
  }
  if (!key_valid) return;
  // dk[mb] / dv[mb] lane (g4, j16) holds d = 16 mb + 4 g4 + i of key mykey: 8-byte stores
  if (run.dk) {
    bf16* p = (bf16*)run.dk + (int64_t)mykey * run.dk_row_stride + (int64_t)hk * run.dk_head_stride + 4 * (lane >> 4);
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const f32x4 v = dk[mb] * P.scale;
      *reinterpret_cast<u32x2*>(p + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    }
  }
  if (run.dv) {
    bf16* p = (bf16*)run.dv + (int64_t)mykey * run.dv_row_stride + (int64_t)hk * run.dv_head_stride + 4 * (lane >> 4);
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
      *reinterpret_cast<u32x2*>(p + 16 * mb) = u32x2{pack2<E>(dv[mb][0], dv[mb][1]), pack2<E>(dv[mb][2], dv[mb][3])};
  }
}

// ---------------------------------------------------------------------------
// backward dK / dV with the keys split over the waves (head dim 128: GQA
// groups that are not a multiple of 4; head dim 256: 48-key work items, which
// launches with few 64-key items take)
//
// A work-group owns P.kv_block keys (48 or 64) of one run and one KV head;
// wave w owns keys 16 w .. 16 w + 15, their K^T and V^T in registers, and all
// waves walk the same sequence of steps -- every query head of the group,
// then every visible 32-row block -- reading one double-buffered LDS stage:
// the step's Q and dO rows (HD-element rows, 16-byte chunk c of row r at slot
// c ^ tile_swizzle(r & 15)) and the rows' 32 (lse * log2 e, delta) pairs,
// filled by buffer_load ... lds with each wave issuing its share of the
// instructions, one work-group barrier per step.  The buffer resource of a
// tile covers exactly its valid rows, so rows past a segment's end arrive as
// zeros and add nothing (S = dP = 0, statistics (0, 0), hence dS = 0 and a
// zero dO row).  S = Q K^T and dP = dO V^T take the Q/dO rows as A operands;
// dV^T += dO^T P and dK^T += Q^T dS take dO^T / Q^T from ds_read_b64_tr_b16
// (the lane layout of the one-wave-per-head kernel).  A wave past the work
// item's keys (kv_block 48) only issues its DMA share; only steps that cross
// the diagonal are masked.
// ---------------------------------------------------------------------------
template <typename E, int HD, bool DS = false>
__global__ __launch_bounds__(kThreads, 1) void dkdv_split_kernel(ts_attn_problem P, ts_attn_rows Q,
                                                                 ts_attn_rows dO,
                                                                 const float* __restrict__ rowstats,
                                                                 int64_t lse_ld, DsArgs S) {
  static_assert(HD == 128 || HD == 256, "the swizzle needs 16 or 32 chunks per row");
  constexpr int CH = HD / 8;              // 16-byte chunks per row
  constexpr int NKS = HD / 32;            // k-steps of S / dP over the head dim
  constexpr int NMB = HD / 16;            // 16-column blocks of dK / dV
  constexpr int TILE = 32 * HD;           // elements of a 32-row tile
  constexpr int STAGE = 2 * TILE + 512;   // Q, dO, then 1 KB of statistics
  constexpr int RPI = 64 / CH;            // rows one DMA instruction fills (4 or 2)
  constexpr int NDMA = 32 / RPI;          // DMA instructions per tile (8 or 16)
  constexpr int PER_WAVE = NDMA / 4;      // of them issued by each wave
  // dO^T / Q^T blocks whose transposed reads are issued before the softmax
  // (head dim 256: eight, 4.94 -> 4.83 ms on the branch shape), and the
  // read-ahead distance of the rest
  constexpr int NPRE = HD == 256 ? 8 : 4;
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
  const int wk0 = k0 + 16 * wave;  // the wave's first key (run-local)
  const int mykey = wk0 + j16;      // the key column this lane holds
  const bool in_block = 16 * wave < P.kv_block;
  const bool wave_active = in_block && wk0 < run.len;  // wave-uniform
  const bool key_valid = in_block && mykey < run.len;
  const float c = P.scale * kLog2e;
  const int nkb = (run.len + 15) >> 4;  // 16-key blocks of the run
  // the key position the causal mask compares against; dS route: a key past
  // the run is put past every row (2^24 rows), so the mask zeroes its P too
  const int mask_key = mykey + (DS && !key_valid ? (1 << 24) : 0);

  int ro[4], to[8];
  swizzled_offsets<HD>(lane, ro, to);
  // DMA instruction t fills rows RPI t .. RPI t + RPI - 1: lane l the row
  // RPI t + l / CH, slot l % CH with logical chunk (l % CH) ^ tile_swizzle(row);
  // this wave issues t = wave + 4 u.  Byte offsets of the lane's row and chunk.
  int qoff[PER_WAVE], doff[PER_WAVE];
#pragma unroll
  for (int u = 0; u < PER_WAVE; ++u) {
    const int row = RPI * (wave + 4 * u) + lane / CH;
    const int chunk = (lane % CH) ^ tile_swizzle(row & 15);
    qoff[u] = (int)((row * Q.row_stride + chunk * 8) * 2);
    doff[u] = (int)((row * dO.row_stride + chunk * 8) * 2);
  }

  // K^T and V^T operands: kreg[ks] = K[key mykey][32 ks + 8 g4 ..], vreg likewise
  bf16x8 kreg[NKS], vreg[NKS];
  {
    const bf16* kp = (const bf16*)run.k + (int64_t)mykey * run.k_row_stride + (int64_t)hk * run.k_head_stride;
    const bf16* vp = (const bf16*)run.v + (int64_t)mykey * run.v_row_stride + (int64_t)hk * run.v_head_stride;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      kreg[ks] = as_bf16x8(key_valid ? ld16(kp + 32 * ks + 8 * g4) : u32x4{0u, 0u, 0u, 0u});
      vreg[ks] = as_bf16x8(key_valid ? ld16(vp + 32 * ks + 8 * g4) : u32x4{0u, 0u, 0u, 0u});
    }
  }
  f32x4 dk[NMB], dv[NMB];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
    dk[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[mb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // dS route.  The dS block computed by a step is stored by the next one
  // (a step before the next wait for all of this wave's memory operations),
  // to pend_at: this lane's element of the block, or of the workspace's sink
  // block (after every head's part) when the step computed none, so the
  // store needs no branch.  The cursor carries `at`, this lane's element of
  // its step's block, advanced by the row block's block count each step and
  // located afresh only on entering a visit or head.  The bookkeeping is kept
  // in VGPRs, derived from an opaque zero: the kernel's scalar registers are
  // all taken, and scalar spills or reloads of kernel arguments inside the
  // loop would serialize its LDS reads.
  int vzero;
  asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
  const int64_t ds_head = DS ? S.head + vzero : 0;
  bf16* const ds_base = DS ? (bf16*)S.ptr + (vzero + ds_store_offset(lane) / 2) : nullptr;
  bf16* const ds_sink = ds_base + P.hq * ds_head;
  bf16* const ds_lane = ds_base + (int64_t)(wk0 >> 4) * kDsBlock;  // key block wk0 / 16
  bf16* pend_at = ds_sink;
  bf16x8 pend = as_bf16x8(u32x4{0u, 0u, 0u, 0u});
  // step cursor: query head g of the group, then the visit / row block
  struct Cursor {
    int g;
    VisitCursor v;
    bf16* at;  // dS route: this lane's element of the step's dS block
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
    // consumed here, so that no scalar load is outstanding when the next
    // step's LDS reads count their completions
    const int64_t blk = load_uniform(S.visit, run.visit0 + cu.v.vi) / kDsBlock +
                        ds_blocks_before(DsRect{cu.v.off - cu.v.kpos, nkb, cu.v.q_len}, cu.v.r0 >> 5);
    asm volatile("" ::"s"(blk));
    return ds_lane + (int64_t)(hk * group + cu.g) * ds_head + blk * kDsBlock;
  };
  // the step after `cu`; g == group at the end
  auto advance = [&](Cursor cu) -> Cursor {
    // blocks of the row block being left (32-bit: d + row < kv_len)
    int inc = 0;
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
    const int h = hk * group + (live ? cu.g : 0);
    const int64_t row0 = live ? cu.v.q_row0 + cu.v.r0 : 0;
    const bf16* qb = (const bf16*)Q.ptr + row0 * Q.row_stride + (int64_t)h * Q.head_stride;
    const bf16* db = (const bf16*)dO.ptr + row0 * dO.row_stride + (int64_t)h * dO.head_stride;
    const rsrc_t rq = make_rsrc(qb, (uint32_t)(nrows * Q.row_stride * 2));
    const rsrc_t rd = make_rsrc(db, (uint32_t)(nrows * dO.row_stride * 2));
#pragma unroll
    for (int u = 0; u < PER_WAVE; ++u) {
      buffer_dma16(rq, buf + (wave + 4 * u) * 512, qoff[u]);
      buffer_dma16(rd, buf + TILE + (wave + 4 * u) * 512, doff[u]);
    }
    if (wave == 0) {
      // 32 rows x 8 bytes of statistics: lanes 0..15, 16 bytes each (the
      // other lanes read past the resource and write zeros after them)
      const rsrc_t rs = make_rsrc(rowstats + 2 * ((int64_t)h * lse_ld + row0), (uint32_t)(nrows * 8));
      buffer_dma16(rs, buf + 2 * TILE, lane < 16 ? lane * 16 : 0x7ffffff0);
    }
  };

  // one step on the tiles in `cur_buf`; buffer roles fixed per call
  auto step = [&](auto bsel, Cursor& cur, Cursor& nxt) {
    bf16* cur_buf = bsel.value == 0 ? s_b0 : s_b1;
    bf16* nxt_buf = bsel.value == 0 ? s_b1 : s_b0;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's share of the step's tiles has landed
    __syncthreads();                // every wave's share has, and nobody reads nxt_buf any more
    issue(nxt, nxt_buf);
    // dS route: the previous step's dS block, stored a step before the next
    // wait for all of this wave's memory operations (after the DMA, which
    // it would otherwise hold up in the memory queue)
    if constexpr (DS) global_st16(pend_at, as_u32x4(pend));
    const int off = cur.v.off, r0 = cur.v.r0, kpos = cur.v.kpos;
    const int nrows = min(32, cur.v.q_len - r0);
    // the wave's keys are all invisible to this block when its first key is
    // beyond the block's last row
    const bool live = wave_active && kpos + wk0 <= off + r0 + nrows - 1;
    // dS route: this step's destination (block wk0 / 16 of row block r0 / 32,
    // inside the rectangle when the wave computes it; its address was formed
    // at the previous step's tail, off the path from the barrier to the first
    // MFMA)
    if constexpr (DS) pend_at = live ? cur.at : ds_sink;
    if (live) {
      const bf16* tq = cur_buf;
      const bf16* td = cur_buf + TILE;
      const float* sl = reinterpret_cast<const float*>(cur_buf + 2 * TILE);  // [32] (lse2, delta)
      // S = Q K^T, dP = dO V^T: [qb] holds rows 16 qb + 4 g4 + i, key j16
      f32x4 sc[2], dp[2];
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        sc[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
        dp[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
          const bf16x8 aq = as_bf16x8(ld16(tq + ro_of(ro, ks) + 16 * qb * HD));
          const bf16x8 ad = as_bf16x8(ld16(td + ro_of(ro, ks) + 16 * qb * HD));
          sc[qb] = mma16<E>(aq, kreg[ks], sc[qb]);
          dp[qb] = mma16<E>(ad, vreg[ks], dp[qb]);
        }
      // Q/dO row reads two k-steps ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        if (ks + 2 < NKS) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
      }
      u32x2 fa[NMB][2], fb[NMB][2];  // dO^T / Q^T fragments of block mb
#pragma unroll
      for (int mb = 0; mb < NPRE; ++mb) {
        const int o = to_of(to, mb);
        fa[mb][0] = tr_read(td + o);
        fa[mb][1] = tr_read(td + o + 16 * HD);
        fb[mb][0] = tr_read(tq + o);
        fb[mb][1] = tr_read(tq + o + 16 * HD);
      }
      __builtin_amdgcn_sched_barrier(0);
      // P and dS as B operands: slot j = 4 qb + i  <->  row 16 qb + 4 g4 + i
      float pv[8], dsv[8];
      const int lim = off + r0 - kpos - mask_key;  // row rl sees the key iff rl >= -lim
      // wave-uniform: the keys cross the diagonal (or, when dS is stored, the
      // run's end: P of a key past it, whose K row is zero, is exp2(-lse2))
      const bool diag = (kpos + wk0 + 15 > off + r0) | (DS && wk0 + 16 > run.len);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rl = 16 * qb + 4 * g4 + i;
          float p = fast_exp2(sc[qb][i] * c - sl[2 * rl]);
          if (diag && rl + lim < 0) p = 0.f;
          pv[4 * qb + i] = p;
          dsv[4 * qb + i] = p * (dp[qb][i] - sl[2 * rl + 1]);
        }
      const bf16x8 pk = pack8<E>(pv);
      const bf16x8 dsk = pack8<E>(dsv);
      if constexpr (DS) pend = dsk;
      __builtin_amdgcn_sched_barrier(0);
      // dV^T += dO^T P, dK^T += Q^T dS: rows d = 16 mb + 4 g4 + i, column key j16
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        if (mb >= NPRE) {
          const int o = to_of(to, mb);
          fa[mb][0] = tr_read(td + o);
          fa[mb][1] = tr_read(td + o + 16 * HD);
          fb[mb][0] = tr_read(tq + o);
          fb[mb][1] = tr_read(tq + o + 16 * HD);
        }
        dv[mb] = mma16<E>(as_bf16x8(u32x4{fa[mb][0][0], fa[mb][0][1], fa[mb][1][0], fa[mb][1][1]}), pk, dv[mb]);
        dk[mb] = mma16<E>(as_bf16x8(u32x4{fb[mb][0][0], fb[mb][0][1], fb[mb][1][0], fb[mb][1][1]}), dsk, dk[mb]);
      }
      // the remaining dO^T / Q^T reads NPRE blocks ahead of their MFMAs
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
        if (mb + NPRE < NMB) __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
      }
    }
    cur = nxt;
    nxt = advance(nxt);
  };

  Cursor cur{0, first_visit(), ds_sink};
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
  if constexpr (DS)
    global_st16(pend_at, as_u32x4(pend));
  __builtin_amdgcn_s_waitcnt(0);  // the last (empty) DMA has landed before the waves exit
  if (!key_valid) return;
  // lane (g4, j16) holds d = 16 mb + 4 g4 .. + 3 of key mykey: 8-byte stores
  if (run.dk) {
    bf16* p = (bf16*)run.dk + (int64_t)mykey * run.dk_row_stride + (int64_t)hk * run.dk_head_stride + 4 * g4;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
      *reinterpret_cast<u32x2*>(p + 16 * mb) =
          u32x2{pack2<E>(dk[mb][0] * P.scale, dk[mb][1] * P.scale), pack2<E>(dk[mb][2] * P.scale, dk[mb][3] * P.scale)};
  }
  if (run.dv) {
    bf16* p = (bf16*)run.dv + (int64_t)mykey * run.dv_row_stride + (int64_t)hk * run.dv_head_stride + 4 * g4;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb)
      *reinterpret_cast<u32x2*>(p + 16 * mb) = u32x2{pack2<E>(dv[mb][0], dv[mb][1]), pack2<E>(dv[mb][2], dv[mb][3])};
  }
}

template <typename E, int HD>
void launch_dkdv_generic(dim3 grid, const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout,
                         const float* rowstats, int64_t lse_ld, hipStream_t s) {
  ts::TimedLaunch timed_("attention.dkdv_kernel", s);
  hipLaunchKernelGGL((dkdv_kernel<E, HD>), grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld);
}

template <typename E, bool DS>
void launch_dkdv_tuned(dim3 grid, const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout,
                       const float* rowstats, int64_t lse_ld, const DsArgs& S, hipStream_t s) {
  const int group = P.hq / P.hkv;
  ts::TimedLaunch timed_("attention.dkdv_kernel", s);
  if (P.head_dim == 256 && P.kv_block == 64)
    launch_dkdv256<E, DS>(grid, P, q, dout, rowstats, lse_ld, S, s);
  else if (P.head_dim == 256)
    hipLaunchKernelGGL((dkdv_split_kernel<E, 256, DS>), grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, S);
  else if (group % 4 == 0)
    launch_dkdv_wave<E, DS>(grid, P, q, dout, rowstats, lse_ld, S, s);
  else
    hipLaunchKernelGGL((dkdv_split_kernel<E, D, DS>), grid, dim3(kThreads), 0, s, P, q, dout, rowstats, lse_ld, S);
}

template <typename E>
int launch_dkdv_t(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout, const float* rowstats,
                  int64_t lse_ld, const DsArgs* ds, hipStream_t s) {
  const dim3 grid((unsigned)(P.n_kv_work * P.hkv));
  switch (P.head_dim) {
    case 32: launch_dkdv_generic<E, 32>(grid, P, q, dout, rowstats, lse_ld, s); break;
    case 64: launch_dkdv_generic<E, 64>(grid, P, q, dout, rowstats, lse_ld, s); break;
    case 96: launch_dkdv_generic<E, 96>(grid, P, q, dout, rowstats, lse_ld, s); break;
    case 192: launch_dkdv_generic<E, 192>(grid, P, q, dout, rowstats, lse_ld, s); break;
    default:  // 128 and 256
      if (ds)
        launch_dkdv_tuned<E, true>(grid, P, q, dout, rowstats, lse_ld, *ds, s);
      else
        launch_dkdv_tuned<E, false>(grid, P, q, dout, rowstats, lse_ld, DsArgs{}, s);
  }
  return ts::check_launch("ts_attn_bwd (dkdv)");
}

int launch_dkdv(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout, const float* rowstats,
                int64_t lse_ld, const DsArgs* ds, hipStream_t s) {
  return P.dtype == kF16 ? launch_dkdv_t<f16>(P, q, dout, rowstats, lse_ld, ds, s)
                         : launch_dkdv_t<bf16>(P, q, dout, rowstats, lse_ld, ds, s);
}

}  // namespace attn
}  // namespace ts
