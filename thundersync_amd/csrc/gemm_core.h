// MFMA GEMM core for gfx950: one 256 x 256 work-group tile of C = A . B^T
// (bf16 or fp16 operands E, fp32 accumulation), shared by the logprob and LoRA kernels.
//
// 8 waves of 128 x 64 (two per SIMD, so one wave's memory instructions overlap
// the other's MFMAs), v_mfma_f32_32x32x16_bf16.  K streams 32 at a time
// through a 4-stage LDS ring filled by buffer_load ... lds (no register
// staging), refilled three stages ahead of the MFMAs, one work-group barrier
// per stage; each barrier also certifies the next stage, whose first
// fragments are read during the current stage's last MFMAs.  An operand is
// either K-contiguous (its rows are the tile's M or N index) or K-strided
// (its rows are the contraction index: read through transposed LDS reads).
// Rows past an operand's valid rows and 8-element K chunks past K arrive as
// zeros (buffer range checking), so ragged edges need no masking in the loop.
#pragma once

#include <type_traits>

#include "common.h"

namespace ts {
namespace gemm {

#ifndef TS_GEMM_WAVES
#define TS_GEMM_WAVES 8
#endif
// waves per work-group: 8 (two per SIMD, wave tile 128 x 64) or 4 (one per
// SIMD, wave tile 128 x 128); wave w covers A rows 128 (w & 1) .. and B rows
// 32 NI (w >> 1) ..
constexpr int kWaves = TS_GEMM_WAVES;
static_assert(kWaves == 8 || kWaves == 4, "8 or 4 waves per GEMM work-group");
constexpr int kGemmThreads = 64 * kWaves;
constexpr int NI = 16 / kWaves;         // 32-column B blocks per wave
constexpr int kDmaPerWave = 16 / kWaves;  // DMA instructions per operand, wave and stage
constexpr int TM = 256;  // A rows (vocab rows, or hidden dims) per work-group
constexpr int TN = 256;  // B rows (tokens) per work-group
constexpr int TK = 32;   // K per LDS stage
constexpr int kStageElems = (TM + TN) * TK;  // 32 KB: A [TM][TK], then B [TN][TK]

__device__ __forceinline__ u32x4 ld16(const bf16* p) { return *reinterpret_cast<const u32x4*>(p); }

// Work-groups are dispatched round-robin over the 8 XCDs; renumber them so each
// XCD runs a contiguous range of logical tiles.
__device__ __forceinline__ int xcd_logical(int bid, int total) {
  const int per = total / 8, rem = total % 8;
  const int xcd = bid % 8, local = bid / 8;
  return xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
}

// Logical tile -> (A tile, B tile) in groups of 4 A tiles: consecutive ids walk
// the B tiles of a group with its 4 A tiles innermost, so the ~32 work-groups
// an XCD runs at once cover 4 A panels x ~8 B panels and share both in L2.
__device__ __forceinline__ void grouped_tile(int id, int n_a, int n_b, int& ta, int& tb) {
  constexpr int G = 4;
  const int g = id / (G * n_b);
  const int r = id - g * G * n_b;
  const int ga = min(G, n_a - g * G);
  tb = r / ga;
  ta = g * G + (r - tb * ga);
}

// One operand's share of a stage: 256 rows x 64 bytes = 16 instructions of 16
// rows each, issued by the waves as t = wave + kWaves u.  Lane i of an
// instruction fills row 16 t + i / 4, slot i & 3 with the logical 16-byte
// chunk c = (i & 3) ^ (i >> 4): row r's chunk c sits at slot c ^ ((r >> 2) & 3),
// so the 16 rows of a fragment read at one chunk hit 16 distinct bank groups.
struct Streamer {
  const bf16* base;  // row 0, k 0
  int64_t ld;
  int rows;          // valid rows from base (>= 1)
  int K;
  int voff[kDmaPerWave];  // byte offset of this lane's row and chunk within a stage, per u
  int kchunk;        // this lane's chunk start within a stage (elements)
  __device__ __forceinline__ void init(const bf16* b, int64_t ld_, int rows_, int K_, int wave, int lane) {
    base = b;
    ld = ld_;
    rows = rows_;
    K = K_;
    kchunk = 8 * ((lane & 3) ^ (lane >> 4));
#pragma unroll
    for (int u = 0; u < kDmaPerWave; ++u)
      voff[u] = (int)(((16 * (wave + kWaves * u) + (lane >> 2)) * ld + kchunk) * 2);
  }
  // descriptor and this lane's chunk validity for K columns [k0, k0 + TK)
  __device__ __forceinline__ u32x4 descriptor(int k0) const {
    return raw_descriptor(base + k0, (uint32_t)(((int64_t)(rows - 1) * ld + TK) * 2));
  }
  // instruction u of this wave's share of the stage into dst (wave-uniform);
  // a chunk past K reads nothing: zeros
  __device__ __forceinline__ void issue(u32x4 r, bool in_k, bf16* dst, int u, int wave) const {
    buffer_dma16_untracked(r, dst + (wave + kWaves * u) * 512, in_k ? voff[u] : 0x7ffffff0);
  }
};

// An operand stored with its contraction index as the row index ("K-strided":
// W read as W^T, dlogits or hidden read as their transposes): the tile's 256
// M values of one K row are contiguous.  A stage holds K rows k0 .. k0 + 31 as
// [32][256] (512-byte rows), 16-byte chunk c of row k at slot c ^ (4 (k & 3)),
// so that the transposed fragment reads below touch 16 distinct bank groups
// per pass.  One instruction moves two K rows: lane i fills row
// 2 t + (i >> 5), slot i & 31, with logical chunk (i & 31) ^ (4 (row & 3)).
// K rows past K and chunks past the operand's end arrive as zeros (buffer
// range checking); chunks past M in earlier rows read the next row, which
// lands in output rows or columns the epilogue discards.
struct StreamerT {
  const bf16* base;  // k 0, m 0 of the tile
  int64_t ld;        // elements between consecutive K rows
  int mvalid;        // valid M columns from base (>= 1)
  int K;
  int voff[kDmaPerWave];
  __device__ __forceinline__ void init(const bf16* b, int64_t ld_, int mvalid_, int K_, int wave, int lane) {
    base = b;
    ld = ld_;
    mvalid = min(mvalid_, TM);
    K = K_;
#pragma unroll
    for (int u = 0; u < kDmaPerWave; ++u) {
      const int row = 2 * (wave + kWaves * u) + (lane >> 5);
      const int c = (lane & 31) ^ (4 * (row & 3));
      voff[u] = (int)((row * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ u32x4 descriptor(int k0) const {
    const int rows = min(TK, K - k0);
    return raw_descriptor(base + (int64_t)k0 * ld, (uint32_t)(((int64_t)(rows - 1) * ld + mvalid) * 2));
  }
  __device__ __forceinline__ void issue(u32x4 r, bf16* dst, int u, int wave) const {
    buffer_dma16_untracked(r, dst + (wave + kWaves * u) * 512, voff[u]);
  }
};

typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 tr_read(const bf16* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  u32x2 r;
  __builtin_memcpy(&r, &v, 8);
  return r;
}

// Fragment reads of one operand of v_mfma_f32_32x32x16_bf16 from a stage part:
// lane l holds M row (l & 31) of a 32-row block and the 8 K values
// 16 kk + 8 (l >> 5) .. + 7 of k-step kk.
//  K-contiguous part ([256 rows][32 k]): one 16-byte read at row, chunk
//    2 kk + (l >> 5), slot chunk ^ ((row >> 2) & 3).
//  K-strided part ([32 k][256 m]): two ds_read_b64_tr_b16.  Within each
//    16-lane group, lane j addressing K row kb + j / 4 at M columns
//    m0 + 4 (j & 3) .. + 3 receives the 4 values at K rows kb .. kb + 3 of
//    column m0 + j (lane semantics pinned by the LDS probe test), so the
//    group g = l >> 4 takes M columns 16 (g & 1) + 0..15 of the block and K
//    rows 16 kk + 8 (g >> 1) + {0..3, 4..7}.
template <bool KS> struct Frag;
template <> struct Frag<false> {
  int off[2];  // per kk, block 0
  __device__ __forceinline__ void init(int lane, int row0) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int slot = ((2 * kk + (lane >> 5)) ^ ((lane >> 2) & 3)) << 3;
      off[kk] = (row0 + (lane & 31)) * TK + slot;
    }
  }
  __device__ __forceinline__ bf16x8 read(const bf16* part, int kk, int blk) const {
    return as_bf16x8(ld16(part + off[kk] + 32 * blk * TK));
  }
};
template <> struct Frag<true> {
  int off[4];  // per 32-row block (kk = 0, first read)
  __device__ __forceinline__ void init(int lane, int row0) {
    const int j = lane & 15, g = lane >> 4;
    const int k = 8 * (g >> 1) + (j >> 2);  // k & 3 == (j >> 2) & 3
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int m = row0 + 32 * b + 16 * (g & 1) + 4 * (j & 3);
      off[b] = k * TM + ((((m >> 3) ^ (4 * (k & 3))) & (TM / 8 - 1)) << 3) + (m & 7);
    }
  }
  __device__ __forceinline__ bf16x8 read(const bf16* part, int kk, int blk) const {
    const u32x2 lo = tr_read(part + off[blk] + 16 * kk * TM);
    const u32x2 hi = tr_read(part + off[blk] + (16 * kk + 4) * TM);
    return as_bf16x8(u32x4{lo[0], lo[1], hi[0], hi[1]});
  }
};

// acc[mi][ni]: 32x32 block (A rows 128 wm + 32 mi, B rows 32 NI wn + 32 ni),
// wm = wave & 1, wn = wave >> 1.  Lane l holds B row b_row(ni, l, wn) and A rows
// a_row(mi, i, l, wm), i = 0..15.
__device__ __forceinline__ int a_row(int mi, int i, int lane, int wm) {
  return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3) + 32 * mi + 128 * wm;
}
__device__ __forceinline__ int b_row(int ni, int lane, int wn) { return 32 * NI * wn + 32 * ni + (lane & 31); }

// The MFMAs of one stage (two k-steps of 16) in a fixed order.  The k-step-0
// fragments a0 / b0 of `st` arrive already in registers (read during the
// previous stage); four groups of {two k-step-0 MFMAs, one or two k-step-1
// fragment reads, one refill DMA instruction}, then the 8 k-step-1 MFMAs,
// beside which the k-step-0 fragments of the next stage `nx` (if any) are
// read into a0 / b0.  Spreading the refill over the MFMAs keeps the wave
// issuing MFMAs while the DMA is in flight, and with the next stage's first
// fragments in registers the MFMAs start right after the stage barrier
// instead of waiting for LDS reads every wave issues at once.
template <typename E, bool HAS_NEXT, class FA, class FB, class Dma>
__device__ __forceinline__ void mma_stage(f32x16 acc[4][NI], const bf16* st, const bf16* nx, const FA& fa,
                                          const FB& fb, bf16x8 (&a0)[4], bf16x8 (&b0)[NI], Dma&& dma) {
  bf16x8 a1[4], b1[NI];
  const bf16* sb = st + TM * TK;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[g][ni] = mma32<E>(a0[g], b0[ni], acc[g][ni]);
    if constexpr (NI == 2) {
      if (g < 2) {
        a1[2 * g] = fa.read(st, 1, 2 * g);
        a1[2 * g + 1] = fa.read(st, 1, 2 * g + 1);
      } else {
        b1[g - 2] = fb.read(sb, 1, g - 2);
      }
    } else {
      a1[g] = fa.read(st, 1, g);
      b1[g] = fb.read(sb, 1, g);
    }
    dma(g);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mma32<E>(a1[mi], b1[ni], acc[mi][ni]);
    if (HAS_NEXT || nx != nullptr) {
      a0[mi] = fa.read(nx, 0, mi);
      if (mi < NI) b0[mi] = fb.read(nx + TM * TK, 0, mi);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// wait until at most `ahead` stages of this wave's DMA instructions are in
// flight (2 kDmaPerWave instructions per stage)
__device__ __forceinline__ void wait_dma(int ahead) {
  if constexpr (kDmaPerWave == 2) {
    if (ahead >= 2) __builtin_amdgcn_s_waitcnt(0x0F78);       // vmcnt(8)
    else if (ahead == 1) __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
    else __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
  } else {
    if (ahead >= 2) __builtin_amdgcn_s_waitcnt(0x4F70);       // vmcnt(16)
    else if (ahead == 1) __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
    else __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
  }
}

// C tile = A . B^T over K through the LDS ring s0..s3 (distinct arrays, so the
// compiler sees that a refill and the reads of another stage never alias);
// the ring is free on return.  AKS / BKS: the operand is K-strided (A is then
// given as its [K][M] storage from the tile's first column, B likewise);
// otherwise K-contiguous (a_rows / b_rows valid rows of 256 from A / B).
template <typename E, bool AKS, bool BKS>
__device__ __forceinline__ void gemm_tile(f32x16 acc[4][NI], const bf16* A, int64_t lda, int a_rows,
                                          const bf16* B, int64_t ldb, int b_rows, int K, bf16* s0,
                                          bf16* s1, bf16* s2, bf16* s3) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.f;
  std::conditional_t<AKS, StreamerT, Streamer> sa;
  std::conditional_t<BKS, StreamerT, Streamer> sb;
  sa.init(A, lda, a_rows, K, wave, lane);
  sb.init(B, ldb, b_rows, K, wave, lane);
  Frag<AKS> fa;
  Frag<BKS> fb;
  fa.init(lane, 128 * wm);
  fb.init(lane, 32 * NI * wn);
  const int nk = (K + TK - 1) / TK;
  // operand s of stage kt: descriptor, and per lane whether its chunk is in K
  // (K-strided operands bound K by the descriptor's row count instead)
  auto in_k = [&](const auto& s, int k0) {
    if constexpr (std::is_same_v<std::decay_t<decltype(s)>, Streamer>) return k0 + s.kchunk < K;
    else return true;
  };
  auto put = [&](const auto& s, u32x4 r, bool ik, bf16* dst, int u) {
    if constexpr (std::is_same_v<std::decay_t<decltype(s)>, Streamer>) s.issue(r, ik, dst, u, wave);
    else s.issue(r, dst, u, wave);
  };
  auto issue = [&](bf16* st, int kt) {
    const u32x4 ra = sa.descriptor(kt * TK), rb = sb.descriptor(kt * TK);
    const bool ka = in_k(sa, kt * TK), kb = in_k(sb, kt * TK);
#pragma unroll
    for (int u = 0; u < kDmaPerWave; ++u) {
      put(sa, ra, ka, st, u);
      put(sb, rb, kb, st + TM * TK, u);
    }
  };
  issue(s0, 0);
  if (nk > 1) issue(s1, 1);
  if (nk > 2) issue(s2, 2);
  // stage 0 landed everywhere: its k-step-0 fragments into registers
  bf16x8 a0[4], b0[NI];
  wait_dma(min(nk - 1, 2));
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) a0[mi] = fa.read(s0, 0, mi);
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) b0[ni] = fb.read(s0 + TM * TK, 0, ni);
  // step kt: this wave's DMA of stages kt and kt + 1 has landed (stage kt + 2
  // may still be in flight); the barrier makes every wave's share of them
  // visible -- the next stage's first fragments are read during this step --
  // and certifies that all waves are done with the stage refilled next (read
  // during step kt - 1 only)
  // A FULL step (kt + 4 < nk) has a next stage and refills a stage that lies
  // wholly inside K, so its body has no branch: the refill DMA and the next
  // stage's fragment reads sit in the MFMAs' basic block.  The last steps
  // take the general form.
  auto step = [&](auto full, const bf16* cur, const bf16* nxt, bf16* refill, int kt) {
    constexpr bool FULL = decltype(full)::value;
    __builtin_amdgcn_sched_barrier(0);  // keep each stage's loads inside its stage
    if constexpr (FULL) wait_dma(1);
    else wait_dma(max(min(nk - 2 - kt, 1), 0));
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    const bool refill_now = FULL || kt + 3 < nk;
    const int k0 = (kt + 3) * TK;
    const u32x4 ra = sa.descriptor(refill_now ? k0 : 0), rb = sb.descriptor(refill_now ? k0 : 0);
    const bool ka = FULL || in_k(sa, k0), kb = FULL || in_k(sb, k0);
    mma_stage<E, FULL>(acc, cur, (FULL || kt + 1 < nk) ? nxt : nullptr, fa, fb, a0, b0, [&](int g) {
      if (refill_now) {
        if constexpr (kDmaPerWave == 2) {
          if (g < 2) put(sa, ra, ka, refill, g);
          else put(sb, rb, kb, refill + TM * TK, g - 2);
        } else {
          put(sa, ra, ka, refill, g);
          put(sb, rb, kb, refill + TM * TK, g);
        }
      }
    });
  };
  constexpr std::true_type full{};
  constexpr std::false_type general{};
  int kt = 0;
  for (; kt + 7 < nk; kt += 4) {
    step(full, s0, s1, s3, kt);
    step(full, s1, s2, s0, kt + 1);
    step(full, s2, s3, s1, kt + 2);
    step(full, s3, s0, s2, kt + 3);
  }
  for (; kt + 4 <= nk; kt += 4) {
    step(general, s0, s1, s3, kt);
    step(general, s1, s2, s0, kt + 1);
    step(general, s2, s3, s1, kt + 2);
    step(general, s3, s0, s2, kt + 3);
  }
  if (kt < nk) step(general, s0, s1, s3, kt);
  if (kt + 1 < nk) step(general, s1, s2, s0, kt + 1);
  if (kt + 2 < nk) step(general, s2, s3, s1, kt + 2);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
}

// the work-group's LDS: the GEMM ring (4 stages, each with 2 KB of slack so
// that a quarter of a staged output tile fits one stage), reused by the
// epilogues
constexpr int kRingElems = kStageElems + 1024;
#define GEMM_RING                                                    \
  __shared__ __attribute__((aligned(16))) bf16 s0[kRingElems];     \
  __shared__ __attribute__((aligned(16))) bf16 s1[kRingElems];     \
  __shared__ __attribute__((aligned(16))) bf16 s2[kRingElems];     \
  __shared__ __attribute__((aligned(16))) bf16 s3[kRingElems];

}  // namespace gemm
}  // namespace ts
