// Attention backward, dS route: dQ = scale * dS K from the dS blocks the
// dK/dV kernel stored (head dims 128 and 256).
//
// A work-group owns the work item's 128 / GC query rows of one segment for GC
// query heads of one GQA group: wave w takes head w % GC and the 32-row block
// w / GC, so the four waves share the K tiles of their KV head (KT keys: 32 at
// head dim 128, 64 at 256).  Each tile step streams, by buffer DMA into an
// LDS stage, the K tile (rows of HD elements, 16-byte chunk c of row r at slot
// c ^ tile_swizzle(r & 15)) and every wave's KT / 16 dS blocks for its row
// block and the tile's 16-key blocks (the rectangle's prefix its rows see:
// blocks past it arrive as zeros, as do K rows past the run).  Per 32 keys of
// the tile,
//     dQ^T[d][slot] += K^T[d][key] dS^T[key][slot]
// with K^T from ds_read_b64_tr_b16 over the K tile (lane (g4, j16): keys
// 4 g4 + t and 16 + 4 g4 + t of column d = 16 mb + j16) and dS^T from the same
// transposed read over the blocks (keys 4 g4 + t of slot 16 mb' + j16): the two
// operands order the 32 keys alike, and the output columns are the blocks'
// row slots.  dS is zero wherever a row does not see a key, so no masking.
// Memory-bound on the dS stream: NST stages keep NST - 1 tiles in flight.  At
// head dim 128 a stage of 32-key tiles is 16 KB, so four work-groups share a
// CU (against two with 64-key tiles: C2 dQ 1.04 -> 0.99 ms); more independent
// work-groups hide each other's waits better than deeper stages do.
// The DMA is issued untracked by the compiler (its waits would otherwise
// cover the stage being filled as well as the one being read): each step
// waits for its own tile with an explicit vmcnt and a work-group barrier.
#include "attention_impl.h"

namespace ts {
namespace attn {

// the K half of issue_kv_tile: a KT-key K tile, each of the WV waves its
// share of the DMA instructions (rows past the run arrive as zeros)
template <int HD, int KT, int WV>
__device__ __forceinline__ void issue_k_tile(int wave, int lane, const TileCursor& tc, bf16* sk) {
  constexpr int CH = HD / 8, RPI = 64 / CH, NI = KT / RPI;
  static_assert(NI % WV == 0, "every wave issues the same number of instructions");
  const int nvalid = min(KT, tc.len - tc.kt0);
  const u32x4 rk = raw_descriptor(tc.kt, (uint32_t)(nvalid * tc.k_rs * 2));
#pragma unroll
  for (int u = 0; u < NI / WV; ++u) {
    const int t = wave + WV * u;
    const int row = RPI * t + lane / CH;
    const int chunk = ((lane % CH) ^ tile_swizzle(row & 15)) << 3;
    buffer_dma16_untracked(rk, sk + t * 512, (row * tc.k_rs + chunk) * 2);
  }
}

// wait until at most N vector-memory instructions of this wave are outstanding
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

#ifndef TS_DQDS_KT128
#define TS_DQDS_KT128 32
#endif
#ifndef TS_DQDS_KT256
#define TS_DQDS_KT256 32
#endif
// keys per K tile: TS_DQDS_KT256 (32: two 24 KB stages, three work-groups per
// CU; against 64-key tiles in three 48 KB stages at one per CU, branch-shape
// dQ 1.04 -> 0.90 ms) at head dim 256, TS_DQDS_KT128 (32) at 128
template <int HD> constexpr int dq_ds_tile_keys() { return HD > 128 ? TS_DQDS_KT256 : TS_DQDS_KT128; }
#ifndef TS_DQDS_ST128
#define TS_DQDS_ST128 2
#endif
#ifndef TS_DQDS_ST128_8
#define TS_DQDS_ST128_8 2
#endif
// LDS stages: three of 48 KB at head dim 256 with 64-key tiles, else
// TS_DQDS_ST128 (two) at head dim 128 (TS_DQDS_ST128_8 for eight-wave
// work-groups) and two at 256
template <int HD, int WV = 4> constexpr int dq_ds_stages() {
  return HD > 128 ? (dq_ds_tile_keys<HD>() == 64 ? 3 : 2) : (WV == 8 ? TS_DQDS_ST128_8 : TS_DQDS_ST128);
}
// work-groups per CU the LDS stages of WV-wave work-groups allow (160 KB per
// CU, at most four, and at most 16 waves)
template <int HD, int WV> constexpr int dq_ds_occupancy() {
  constexpr int stage = (dq_ds_tile_keys<HD>() * HD + WV * (dq_ds_tile_keys<HD>() / 16) * kDsBlock) * 2;
  constexpr int n = (160 * 1024) / (dq_ds_stages<HD, WV>() * stage);
  constexpr int cap = 16 / WV;
  return n > cap ? cap : n;
}

// WV waves (4, or 8 at head dim 128 with GC = 4 over 64-row items)
template <typename E, int HD, int GC, int WV = 4>
__global__ __launch_bounds__(64 * WV, (dq_ds_occupancy<HD, WV>())) void dq_ds_kernel(ts_attn_problem P, DsArgs S,
                                                                                     ts_attn_rows dQ) {
  static_assert(HD == 128 || HD == 256, "the K tile swizzle needs 16 or 32 chunks per row");
  constexpr int KT = dq_ds_tile_keys<HD>();      // keys per tile (64 or 32)
  constexpr int NKB = KT / 16;                   // 16-key dS blocks per tile
  constexpr int NMB = HD / 16;                   // 16-column blocks of dQ
  constexpr int NST = dq_ds_stages<HD, WV>();    // LDS stages
  constexpr int KTILE = KT * HD;                 // elements of a K tile
  constexpr int DTILE = NKB * kDsBlock;          // a wave's dS blocks of the tile
  constexpr int STAGE = KTILE + WV * DTILE;
  constexpr int PER_TILE = KT * HD / 512 / WV + NKB;  // DMA instructions per wave and tile
  __shared__ __attribute__((aligned(16))) bf16 s_buf[NST * STAGE];
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
  const int rb = (q0 >> 5) + wave / GC;  // this wave's row block
  const ts_attn_segment seg = load_uniform(P.segs, seg_id);
  const int T = seg.q_len;
  const int off = seg.kv_len - seg.q_len;
  const int last = min(q0 + 32 * WV / GC, T) - 1;  // the work-group's last row
  const bool rows_valid = 32 * rb < T;

  int ro[4], to[8];
  swizzled_offsets<HD>(lane, ro, to);
  // transposed-read offsets into a dS block: key 4 g4 + j16 / 4, slots
  // 16 mb' + 4 (j16 & 3) .. + 3 (logical chunk 2 mb' + (j16 & 3) / 2)
  int dso[2];
#pragma unroll
  for (int mbp = 0; mbp < 2; ++mbp) {
    const int kk = 4 * g4 + (j16 >> 2);
    const int lc = 2 * mbp + ((j16 & 3) >> 1);
    dso[mbp] = 32 * kk + ((lc ^ ((kk >> 1) & 2)) << 3) + 4 * (j16 & 1);
  }

  // this wave's dS blocks in the current span: element offset of its row
  // block's first block, and how many blocks it holds
  int ds_sp = -1, ds_n = 0;
  int64_t ds_at = 0;
  auto ds_enter = [&](const TileCursor& tc) {
    ds_sp = tc.sp;
    const int64_t base = load_uniform(S.span, (int64_t)seg.span0 + tc.sp);
    const DsRect R{off - tc.kpos, (tc.len + 15) >> 4, T};
    ds_n = rows_valid ? ds_blocks_in(R, rb) : 0;
    ds_at = (int64_t)h * S.head + base + (rows_valid ? ds_blocks_before(R, rb) : 0) * kDsBlock;
  };
  auto issue = [&](const TileCursor& tc, int st) {
    bf16* buf = s_buf + st * STAGE;
    issue_k_tile<HD, KT, WV>(wave, lane, tc, buf);
    if (tc.sp != ds_sp) ds_enter(tc);
    const int kb0 = tc.kt0 >> 4;
    const int nb = max(0, min(NKB, ds_n - kb0));
    const u32x4 rd = raw_descriptor((const E*)S.ptr + ds_at + (int64_t)kb0 * kDsBlock, (uint32_t)(nb * kDsBlock * 2));
    bf16* dbuf = buf + KTILE + wave * DTILE;
#pragma unroll
    for (int kk = 0; kk < NKB; ++kk) buffer_dma16_untracked_nt(rd, dbuf + kk * kDsBlock, kk * kDsBlock * 2 + lane * 16);
  };

  f32x4 acc[NMB][2];
#pragma unroll
  for (int mb = 0; mb < NMB; ++mb) {
    acc[mb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](int st) {
    const bf16* tk = s_buf + st * STAGE;
    const bf16* td = tk + KTILE + wave * DTILE;
#pragma unroll
    for (int ss = 0; ss < KT / 32; ++ss) {
      bf16x8 b[2];
#pragma unroll
      for (int mbp = 0; mbp < 2; ++mbp) {
        const u32x2 b0 = tr_read(td + 2 * ss * kDsBlock + dso[mbp]);
        const u32x2 b1 = tr_read(td + (2 * ss + 1) * kDsBlock + dso[mbp]);
        b[mbp] = as_bf16x8(u32x4{b0[0], b0[1], b1[0], b1[1]});
      }
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        const u32x2 a0 = tr_read(tk + to_of(to, mb) + 32 * ss * HD);
        const u32x2 a1 = tr_read(tk + to_of(to, mb) + (32 * ss + 16) * HD);
        const bf16x8 a = as_bf16x8(u32x4{a0[0], a0[1], a1[0], a1[1]});
        acc[mb][0] = mma16<E>(a, b[0], acc[mb][0]);
        acc[mb][1] = mma16<E>(a, b[1], acc[mb][1]);
      }
      // K^T reads kept four blocks ahead of their MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
#pragma unroll
      for (int mb = 0; mb < NMB; ++mb) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        if (mb + 4 < NMB) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // tiles i .. i + NST - 2 are in flight at the top of step i
  TileCursor nx = first_kv_tile<KT>(P, seg, hk, last);
  int issued = 0;
#pragma unroll
  for (int p = 0; p < NST - 1; ++p) {
    if (nx.sp < seg.nspan) {
      issue(nx, p);
      nx = next_kv_tile<KT>(P, seg, hk, last, nx);
      ++issued;
    }
  }
  for (int i = 0; i < issued; ++i) {
    // tile i has landed once at most the instructions of the tiles issued
    // after it are outstanding (they complete in issue order)
    const int ahead = issued - 1 - i;
    if (NST > 3 && ahead >= 2)
      wait_vmcnt<2 * PER_TILE>();
    else if (NST > 2 && ahead >= 1)
      wait_vmcnt<PER_TILE>();
    else
      __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // tile i is in every stage; stage (i - 1) % NST is free
    if (nx.sp < seg.nspan) {
      issue(nx, (i + NST - 1) % NST);
      nx = next_kv_tile<KT>(P, seg, hk, last, nx);
      ++issued;
    }
    compute(i % NST);
  }

  if (!rows_valid) return;
  // acc[mb][mb'] lane (g4, j16): d = 16 mb + 4 g4 + i of slot 16 mb' + j16,
  // i.e. of row 32 rb + 16 ((j16 >> 2) & 1) + 4 (2 mb' + (j16 >> 3)) + (j16 & 3)
#pragma unroll
  for (int mbp = 0; mbp < 2; ++mbp) {
    const int row = 32 * rb + 16 * ((j16 >> 2) & 1) + 4 * (2 * mbp + (j16 >> 3)) + (j16 & 3);
    if (row >= T) continue;
    bf16* qrow = (bf16*)dQ.ptr + (seg.q_row0 + row) * dQ.row_stride + (int64_t)h * dQ.head_stride + 4 * g4;
#pragma unroll
    for (int mb = 0; mb < NMB; ++mb) {
      const f32x4 v = acc[mb][mbp] * P.scale;
      *reinterpret_cast<u32x2*>(qrow + 16 * mb) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    }
  }
}

template <typename E, int HD>
void launch_dq_ds_hd(const ts_attn_problem& P, int gc, dim3 grid, const DsArgs& S, ts_attn_rows dq,
                     hipStream_t s) {
  ts::TimedLaunch timed_("attention.dq_kernel", s);
  if (gc == 4)
    hipLaunchKernelGGL((dq_ds_kernel<E, HD, 4>), grid, dim3(kThreads), 0, s, P, S, dq);
  else if (gc == 2)
    hipLaunchKernelGGL((dq_ds_kernel<E, HD, 2>), grid, dim3(kThreads), 0, s, P, S, dq);
  else
    hipLaunchKernelGGL((dq_ds_kernel<E, HD, 1>), grid, dim3(kThreads), 0, s, P, S, dq);
}

template <typename E>
void launch_dq_ds_t(const ts_attn_problem& P, const DsArgs& S, ts_attn_rows dq, hipStream_t s) {
  const int group = P.hq / P.hkv;
  const int gc = heads_per_block(group);
  if (S.dq_work && P.head_dim == 128 && gc == 4) {
    // 64-row items: eight waves, two 32-row blocks per head
    ts_attn_problem P2 = P;
    P2.q_work = S.dq_work;
    P2.n_q_work = S.n_dq_work;
    P2.n_q_long = S.n_dq_long;
    if (P2.n_q_work == 0) return;
    ts::TimedLaunch timed_("attention.dq_kernel", s);
    hipLaunchKernelGGL((dq_ds_kernel<E, 128, 4, 8>), dim3((unsigned)(P2.n_q_work * P.hkv * (group / 4))),
                       dim3(512), 0, s, P2, S, dq);
    return;
  }
  const dim3 grid((unsigned)(P.n_q_work * P.hkv * (group / gc)));
  if (P.head_dim == 256)
    launch_dq_ds_hd<E, 256>(P, gc, grid, S, dq, s);
  else
    launch_dq_ds_hd<E, 128>(P, gc, grid, S, dq, s);
}

int launch_dq_ds(const ts_attn_problem& P, const DsArgs& S, ts_attn_rows dq, hipStream_t s) {
  if (P.dtype == kF16)
    launch_dq_ds_t<f16>(P, S, dq, s);
  else
    launch_dq_ds_t<bf16>(P, S, dq, s);
  return ts::check_launch("ts_attn_bwd (dq from dS)");
}

}  // namespace attn
}  // namespace ts
