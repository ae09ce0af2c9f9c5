// Chunked-vocab fused log-probability / entropy and its gradient with respect
// to the hidden states, for gfx950 (bf16 operands, fp32 accumulation).
//
// Reference: accel/fused_logprob.py:61-338.  The reference materialises one
// fp32 [chunk, V] logit block per chunk and makes several passes over it; here
// the logits never leave the MFMA accumulators:
//
//   forward   logits^T tile = W_tile . H_tile^T on MFMA (A = vocab rows of W,
//             B = token rows of H, both K-contiguous).  The epilogue reduces
//             each token column of the tile to (max, sum exp, sum exp*(l-max))
//             and picks the target logit; a combine kernel merges the per-tile
//             partials into logprob, entropy and lse.  HBM traffic: W once,
//             H once per vocab super-tile, partials (12 bytes/token/tile).
//   backward  the same tile GEMM recomputes the logits; the epilogue forms
//             dlogits = -p (g_lp + g_H (log p + H)) + g_lp [v == t] in
//             registers, rounds it to bf16 (the reference rounds dlogits to the
//             hidden dtype before its VJP GEMM, fused_logprob.py:165, :295) and
//             stores a [rows, V] bf16 block; a second GEMM multiplies it by
//             W (given as W^T so both operands are K-contiguous) into dh.
//
// GEMM core: 256 x 256 work-group tile, 8 waves of 128 x 64 (two per SIMD, so
// one wave's memory instructions overlap the other's MFMAs; accumulators in
// the accumulation registers), v_mfma_f32_32x32x16_bf16.  K streams 32 at a
// time through a 4-stage LDS ring filled by buffer_load ... lds (no register
// staging), refilled three stages ahead of the MFMAs, one work-group barrier
// per stage; each barrier also certifies the next stage, whose first
// fragments are read during the current stage's last MFMAs.
// Rows past an operand's valid rows and 8-element K chunks past K arrive as
// zeros (buffer range checking), so ragged edges need no masking in the loop.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace lp {

constexpr int kThreads = 256;      // combine / transpose kernels
constexpr int kGemmThreads = 512;  // GEMM work-groups: 8 waves, 2 per SIMD
constexpr int NI = 2;              // 32-column B blocks per wave (wave tile 128 x 64)
constexpr int TM = 256;  // A rows (vocab rows, or hidden dims) per work-group
constexpr int TN = 256;  // B rows (tokens) per work-group
constexpr int TK = 32;   // K per LDS stage
constexpr int kStageElems = (TM + TN) * TK;  // 32 KB: A [TM][TK], then B [TN][TK]
constexpr int BM = TM;   // vocab rows per forward partial
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }
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
// rows each, issued by the 8 waves as t = wave + 8 u.  Lane i of an
// instruction fills row 16 t + i / 4, slot i & 3 with the logical 16-byte
// chunk c = (i & 3) ^ (i >> 4): row r's chunk c sits at slot c ^ ((r >> 2) & 3),
// so the 16 rows of a fragment read at one chunk hit 16 distinct bank groups.
struct Streamer {
  const bf16* base;  // row 0, k 0
  int64_t ld;
  int rows;          // valid rows from base (>= 1)
  int K;
  int voff[2];       // byte offset of this lane's row and chunk within a stage, per u
  int kchunk;        // this lane's chunk start within a stage (elements)
  __device__ __forceinline__ void init(const bf16* b, int64_t ld_, int rows_, int K_, int wave, int lane) {
    base = b;
    ld = ld_;
    rows = rows_;
    K = K_;
    kchunk = 8 * ((lane & 3) ^ (lane >> 4));
#pragma unroll
    for (int u = 0; u < 2; ++u) voff[u] = (int)(((16 * (wave + 8 * u) + (lane >> 2)) * ld + kchunk) * 2);
  }
  // descriptor and this lane's chunk validity for K columns [k0, k0 + TK)
  __device__ __forceinline__ u32x4 descriptor(int k0) const {
    return raw_descriptor(base + k0, (uint32_t)(((int64_t)(rows - 1) * ld + TK) * 2));
  }
  // instruction u of this wave's share of the stage into dst (wave-uniform);
  // a chunk past K reads nothing: zeros
  __device__ __forceinline__ void issue(u32x4 r, bool in_k, bf16* dst, int u, int wave) const {
    buffer_dma16_untracked(r, dst + (wave + 8 * u) * 512, in_k ? voff[u] : 0x7ffffff0);
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
  int voff[2];
  __device__ __forceinline__ void init(const bf16* b, int64_t ld_, int mvalid_, int K_, int wave, int lane) {
    base = b;
    ld = ld_;
    mvalid = min(mvalid_, TM);
    K = K_;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int row = 2 * (wave + 8 * u) + (lane >> 5);
      const int c = (lane & 31) ^ (4 * (row & 3));
      voff[u] = (int)((row * ld + 8 * c) * 2);
    }
  }
  __device__ __forceinline__ u32x4 descriptor(int k0) const {
    const int rows = min(TK, K - k0);
    return raw_descriptor(base + (int64_t)k0 * ld, (uint32_t)(((int64_t)(rows - 1) * ld + mvalid) * 2));
  }
  __device__ __forceinline__ void issue(u32x4 r, bf16* dst, int u, int wave) const {
    buffer_dma16_untracked(r, dst + (wave + 8 * u) * 512, voff[u]);
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

// acc[mi][ni]: 32x32 block (A rows 128 wm + 32 mi, B rows 64 wn + 32 ni),
// wm = wave & 1, wn = wave >> 1.  Lane l holds B row (l & 31) + 32 ni + 64 wn and A rows
// 8 (i >> 2) + 4 (l >> 5) + (i & 3) + 32 mi + 128 wm, i = 0..15.
__device__ __forceinline__ int a_row(int mi, int i, int lane, int wm) {
  return 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3) + 32 * mi + 128 * wm;
}

// The MFMAs of one stage (two k-steps of 16) in a fixed order.  The k-step-0
// fragments a0 / b0 of `st` arrive already in registers (read during the
// previous stage); four groups of {two k-step-0 MFMAs, one or two k-step-1
// fragment reads, one refill DMA instruction}, then the 8 k-step-1 MFMAs,
// beside which the k-step-0 fragments of the next stage `nx` (if any) are
// read into a0 / b0.  Spreading the refill over the MFMAs keeps the wave
// issuing MFMAs while the DMA is in flight, and with the next stage's first
// fragments in registers the MFMAs start right after the stage barrier
// instead of waiting for LDS reads every wave issues at once.
template <class FA, class FB, class Dma>
__device__ __forceinline__ void mma_stage(f32x16 acc[4][NI], const bf16* st, const bf16* nx, const FA& fa,
                                          const FB& fb, bf16x8 (&a0)[4], bf16x8 (&b0)[NI], Dma&& dma) {
  bf16x8 a1[4], b1[NI];
  const bf16* sb = st + TM * TK;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    acc[g][0] = mfma32(a0[g], b0[0], acc[g][0]);
    acc[g][1] = mfma32(a0[g], b0[1], acc[g][1]);
    if (g < 2) {
      a1[2 * g] = fa.read(st, 1, 2 * g);
      a1[2 * g + 1] = fa.read(st, 1, 2 * g + 1);
    } else {
      b1[g - 2] = fb.read(sb, 1, g - 2);
    }
    dma(g);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = mfma32(a1[mi], b1[ni], acc[mi][ni]);
    if (nx != nullptr) {
      a0[mi] = fa.read(nx, 0, mi);
      if (mi < NI) b0[mi] = fb.read(nx + TM * TK, 0, mi);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// wait until at most 4 * ahead of this wave's DMA instructions are in flight
__device__ __forceinline__ void wait_dma(int ahead) {
  if (ahead >= 2) __builtin_amdgcn_s_waitcnt(0x0F78);       // vmcnt(8)
  else if (ahead == 1) __builtin_amdgcn_s_waitcnt(0x0F74);  // vmcnt(4)
  else __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
}

// C tile = A . B^T over K through the LDS ring s0..s3 (distinct arrays, so the
// compiler sees that a refill and the reads of another stage never alias);
// the ring is free on return.  AKS / BKS: the operand is K-strided (A is then
// given as its [K][M] storage from the tile's first column, B likewise);
// otherwise K-contiguous (a_rows / b_rows valid rows of 256 from A / B).
template <bool AKS, bool BKS>
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
  fb.init(lane, 64 * wn);
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
    for (int u = 0; u < 2; ++u) {
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
  auto step = [&](const bf16* cur, const bf16* nxt, bf16* refill, int kt) {
    __builtin_amdgcn_sched_barrier(0);  // keep each stage's loads inside its stage
    wait_dma(max(min(nk - 2 - kt, 1), 0));
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    const bool refill_now = kt + 3 < nk;
    const int k0 = (kt + 3) * TK;
    const u32x4 ra = sa.descriptor(refill_now ? k0 : 0), rb = sb.descriptor(refill_now ? k0 : 0);
    const bool ka = in_k(sa, k0), kb = in_k(sb, k0);
    mma_stage(acc, cur, kt + 1 < nk ? nxt : nullptr, fa, fb, a0, b0, [&](int g) {
      if (refill_now) {
        if (g < 2) put(sa, ra, ka, refill, g);
        else put(sb, rb, kb, refill + TM * TK, g - 2);
      }
    });
  };
  int kt = 0;
  for (; kt + 4 <= nk; kt += 4) {
    step(s0, s1, s3, kt);
    step(s1, s2, s0, kt + 1);
    step(s2, s3, s1, kt + 2);
    step(s3, s0, s2, kt + 3);
  }
  if (kt < nk) step(s0, s1, s3, kt);
  if (kt + 1 < nk) step(s1, s2, s0, kt + 1);
  if (kt + 2 < nk) step(s2, s3, s1, kt + 2);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();
}

// the work-group's LDS: the GEMM ring (4 stages, each with 2 KB of slack so
// that a quarter of a staged output tile fits one stage), reused by the
// epilogues
constexpr int kRingElems = kStageElems + 1024;
#define LP_RING                                                    \
  __shared__ __attribute__((aligned(16))) bf16 s0[kRingElems];     \
  __shared__ __attribute__((aligned(16))) bf16 s1[kRingElems];     \
  __shared__ __attribute__((aligned(16))) bf16 s2[kRingElems];     \
  __shared__ __attribute__((aligned(16))) bf16 s3[kRingElems];

// (max, sum exp(l - max), sum exp(l - max) (l - max)) of two disjoint sets of
// logits, either of which may be empty (max = -inf)
__device__ __forceinline__ void merge_stats(float& m, float& s, float& e, float mo, float so, float eo) {
  if (mo == neg_inf()) return;
  if (m == neg_inf()) {
    m = mo;
    s = so;
    e = eo;
    return;
  }
  const float mn = fmaxf(m, mo);
  const float a = fast_exp2((m - mn) * kLog2e);
  const float b = fast_exp2((mo - mn) * kLog2e);
  e = a * (e + s * (m - mn)) + b * (eo + so * (mo - mn));
  s = a * s + b * so;
  m = mn;
}

// ---------------------------------------------------------------------------
// forward: per (vocab tile, token tile) partial softmax statistics
// ---------------------------------------------------------------------------
struct FwdArgs {
  const bf16* h;
  int64_t ldh;
  const bf16* w;
  int64_t ldw;
  const int64_t* target;
  int rows, dim, vocab;
  int n_ttiles, n_vtiles;
  float* part_m;   // [n_vtiles][rows]
  float* part_s;
  float* part_e;
  float* tgt;      // [rows] target logit
};

__global__ __launch_bounds__(kGemmThreads, 1) void fwd_stats_kernel(FwdArgs p) {
  LP_RING
  const int total = p.n_ttiles * p.n_vtiles;
  int vt, tt;
  grouped_tile(xcd_logical(blockIdx.x, total), p.n_vtiles, p.n_ttiles, vt, tt);
  const int v0 = vt * TM, n0 = tt * TN;
  f32x16 acc[4][NI];
  gemm_tile<false, false>(acc, p.w + (int64_t)v0 * p.ldw, p.ldw, min(TM, p.vocab - v0),
                          p.h + (int64_t)n0 * p.ldh, p.ldh, min(TN, p.rows - n0), p.dim, s0, s1, s2, s3);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  float* xm = reinterpret_cast<float*>(s0);  // [TN] per token, from the wm = 1 waves
  float* xs = xm + TN;
  float* xe = xs + TN;
  // rows past the vocabulary (last vocab tile only) take no part
  if (v0 + TM > p.vocab) {
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          if (v0 + a_row(mi, i, lane, wm) >= p.vocab) acc[mi][ni][i] = neg_inf();
  }
  float mk[NI], sk[NI], ek[NI];  // this lane's column statistics, kept across the exchange
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = 64 * wn + 32 * ni + (lane & 31);
    float m = neg_inf();
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; i += 2) m = fmaxf(m, fmaxf(acc[mi][ni][i], acc[mi][ni][i + 1]));
    // sum of q = 2^d2 and of q d2 with d2 = (l - m) log2 e as one FMA per logit; the second
    // sum is taken back to natural-log units once
    float sum = 0.f, e = 0.f;
    const float m2 = m * kLog2e;
    if (v0 + TM <= p.vocab) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float d2 = fmaf(acc[mi][ni][i], kLog2e, -m2);
          const float q = fast_exp2(d2);
          sum += q;
          e = fmaf(q, d2, e);
        }
    } else if (m != neg_inf()) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float d2 = fmaf(acc[mi][ni][i], kLog2e, -m2);  // -inf past the vocabulary: q = 0
          const float q = fast_exp2(d2);
          sum += q;
          e = q > 0.f ? fmaf(q, d2, e) : e;
        }
    }
    e *= kLn2;
    // merge with the other half-wave (lane ^ 32 holds the other vocab rows)
    {
      const float mo = shfl_xor(m, 32), so = shfl_xor(sum, 32), eo = shfl_xor(e, 32);
      merge_stats(m, sum, e, mo, so, eo);
    }
    if (wm == 1 && lane < 32) {
      xm[col] = m;
      xs[col] = sum;
      xe[col] = e;
    }
    mk[ni] = m;
    sk[ni] = sum;
    ek[ni] = e;
  }
  __syncthreads();  // one exchange for both column groups (their columns differ)
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int col = 64 * wn + 32 * ni + (lane & 31);
    const int n = n0 + col;
    if (wm == 0 && lane < 32 && n < p.rows) {
      merge_stats(mk[ni], sk[ni], ek[ni], xm[col], xs[col], xe[col]);
      const int64_t o = (int64_t)vt * p.rows + n;
      p.part_m[o] = mk[ni];
      p.part_s[o] = sk[ni];
      p.part_e[o] = ek[ni];
    }
  }
}

// target logit l[n, t] = sum_d h[n, d] W[t, d] (fp32 sum of exact bf16
// products), one wave per row; rows with t outside [0, vocab) are skipped
// (the combine kernel writes NaN for them)
__global__ __launch_bounds__(kThreads) void target_logit_kernel(const bf16* __restrict__ h, int64_t ldh,
                                                                const bf16* __restrict__ w, int64_t ldw,
                                                                const int64_t* __restrict__ target, int rows,
                                                                int dim, int vocab, float* __restrict__ tgt) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (n >= rows) return;
  const int64_t t = target[n];
  if (t < 0 || t >= vocab) return;
  const bf16* hr = h + (int64_t)n * ldh;
  const bf16* wr = w + t * ldw;
  float acc = 0.f;
  for (int d = 8 * lane; d < dim; d += 512) {
    const u32x4 a = ld16(hr + d), b = ld16(wr + d);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = fmaf(bf_bits_to_f(a[i] & 0xffffu), bf_bits_to_f(b[i] & 0xffffu), acc);
      acc = fmaf(bf_bits_to_f(a[i] >> 16), bf_bits_to_f(b[i] >> 16), acc);
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) tgt[n] = acc;
}

// merge the per-vocab-tile partials of each token: a work-group owns 64 tokens;
// its 4 waves merge the tiles t = wave, wave + 4, ... (lanes read 64
// consecutive tokens of one tile: coalesced), then wave 0 merges the four
// partial states in wave order
__global__ __launch_bounds__(kThreads) void combine_kernel(const float* __restrict__ pm,
                                                           const float* __restrict__ ps,
                                                           const float* __restrict__ pe,
                                                           const float* __restrict__ tgt,
                                                           const int64_t* __restrict__ target,
                                                           int rows, int n_vtiles, int vocab,
                                                           float* __restrict__ logprob,
                                                           float* __restrict__ entropy,
                                                           float* __restrict__ lse) {
  __shared__ float sm[4][64], ss[4][64], se[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = blockIdx.x * 64 + lane;
  float M = neg_inf(), S = 0.f, E = 0.f;  // E: sum exp(l - M) (l - M)
  if (n < rows) {
    for (int t = wave; t < n_vtiles; t += 4) {
      const int64_t o = (int64_t)t * rows + n;
      merge_stats(M, S, E, pm[o], ps[o], pe[o]);
    }
  }
  sm[wave][lane] = M;
  ss[wave][lane] = S;
  se[wave][lane] = E;
  __syncthreads();
  if (wave != 0 || n >= rows) return;
#pragma unroll
  for (int w = 1; w < 4; ++w) merge_stats(M, S, E, sm[w][lane], ss[w][lane], se[w][lane]);
  const float logs = logf(S);
  const int64_t tg = target[n];
  const bool ok = tg >= 0 && tg < vocab;
  logprob[n] = ok ? (tgt[n] - M) - logs : __builtin_nanf("");
  lse[n] = M + logs;
  if (entropy) entropy[n] = logs - E / S;
}

// ---------------------------------------------------------------------------
// backward 1: recompute logits, form bf16 dlogits [rows, ld] (pad columns 0)
// ---------------------------------------------------------------------------
struct DlArgs {
  const bf16* h;
  int64_t ldh;
  const bf16* w;
  int64_t ldw;
  const int64_t* target;
  const float* lse;
  const float* ent;
  const float* g_lp;
  const float* g_ent;  // may be null
  int rows, dim, vocab, vocab_pad;
  int n_ttiles, n_vtiles;
  bf16* dl;
  int64_t ldl;
};

constexpr int OPITCH = TM + 8;  // staging pitch (bf16) of [64 tokens][TM vocab] quarter tiles
static_assert(64 * OPITCH <= kRingElems, "a quarter of the dlogits tile fits one ring stage");

__global__ __launch_bounds__(kGemmThreads, 1) void dlogits_kernel(DlArgs p) {
  LP_RING
  const int total = p.n_ttiles * p.n_vtiles;
  int vt, tt;
  grouped_tile(xcd_logical(blockIdx.x, total), p.n_vtiles, p.n_ttiles, vt, tt);
  const int v0 = vt * TM, n0 = tt * TN;
  f32x16 acc[4][NI];
  gemm_tile<false, false>(acc, p.w + (int64_t)v0 * p.ldw, p.ldw, min(TM, p.vocab - v0),
                          p.h + (int64_t)n0 * p.ldh, p.ldh, min(TN, p.rows - n0), p.dim, s0, s1, s2, s3);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  // tokens 64 q .. 64 q + 63 of the tile are staged in ring stage q as [64][OPITCH]
  auto quarter = [&](int q) -> bf16* { return q == 0 ? s0 : q == 1 ? s1 : q == 2 ? s2 : s3; };
  // dl = -p (g_lp + g_H (log p + H)) + g_lp [v = t], with log2 p = l log2 e - lse log2 e as one
  // FMA and the bracket as one FMA in log2 p: A = g_H ln 2, B = g_lp + g_H H per token.  Tiles
  // inside the vocabulary and the row range (all but the last of each) skip the bounds tests.
  auto epilogue = [&](auto full_c) __attribute__((always_inline)) {
    constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) {
      const int col = 64 * wn + 32 * ni + (lane & 31);  // token within the tile
      bf16* out = quarter(col >> 6) + (col & 63) * OPITCH;
      const int n = n0 + col;
      float lse2 = 0.f, coef_a = 0.f, coef_b = 0.f, glp = 0.f;
      int t = -1;
      if (FULL || n < p.rows) {
        lse2 = p.lse[n] * kLog2e;
        glp = p.g_lp[n];
        coef_b = glp;
        if (p.g_ent) {
          const float gent = p.g_ent[n];
          coef_a = gent * kLn2;
          coef_b = fmaf(gent, p.ent[n], glp);
        }
        const int64_t tt = p.target[n];
        t = (tt >= 0 && tt < p.vocab) ? (int)tt : -1;  // out-of-range targets match no row
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          uint32_t packed[2];
#pragma unroll
          for (int j = 0; j < 4; j += 2) {
            float d2[2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
              const int i = 4 * i4 + j + jj;
              const int v = v0 + a_row(mi, i, lane, wm);
              const float logp2 = fmaf(acc[mi][ni][i], kLog2e, -lse2);
              float d = -fast_exp2(logp2) * fmaf(coef_a, logp2, coef_b);
              if (v == t) d += glp;
              if (!FULL && !(v < p.vocab && n < p.rows)) d = 0.f;
              d2[jj] = d;
            }
            packed[j >> 1] = pack_bf2(d2[0], d2[1]);
          }
          // vocab rows a_row(mi, 4 i4 .. 4 i4 + 3) are consecutive: one 8-byte write
          *reinterpret_cast<u32x2*>(out + a_row(mi, 4 * i4, lane, wm)) = u32x2{packed[0], packed[1]};
        }
    }
  };
  if (v0 + TM <= p.vocab && n0 + TN <= p.rows) epilogue(std::true_type{});
  else epilogue(std::false_type{});
  __syncthreads();
  // coalesced store of the [TN tokens][TM vocab] tile
  const int vmax = min(TM, p.vocab_pad - v0);
#pragma unroll 4
  for (int it = 0; it < (TN * TM / 8) / kGemmThreads; ++it) {
    const int c = it * kGemmThreads + tid;
    const int row = c / (TM / 8), chunk = (c % (TM / 8)) * 8;
    const int n = n0 + row;
    if (n < p.rows && chunk < vmax)
      *reinterpret_cast<u32x4*>(p.dl + (int64_t)n * p.ldl + v0 + chunk) =
          *reinterpret_cast<const u32x4*>(quarter(row >> 6) + (row & 63) * OPITCH + chunk);
  }
}

// ---------------------------------------------------------------------------
// backward 2: grad_hidden[n][d] = sum_v dl[n][v] W[v][d] as C^T = W^T . dl^T,
// W read in place as a K-strided operand (its rows are the contraction
// index).  With `ksplit` > 1 the vocabulary is cut into ksplit ranges of
// whole stages; range s of every tile writes fp32 partial sums to
// part[s][n][d] and grad_hidden_reduce_kernel adds them in range order.
// ---------------------------------------------------------------------------
struct DhArgs {
  const bf16* w;    // [vocab][ldw]
  int64_t ldw;
  const bf16* dl;   // [rows][ldl]
  int64_t ldl;
  int rows, dim, vocab;
  int n_ttiles, n_dtiles, ksplit, kper;  // kper: vocabulary per range (multiple of TK)
  bf16* dh;
  int64_t ldd;
  float* part;      // [ksplit][rows][dim] when ksplit > 1
};

__global__ __launch_bounds__(kGemmThreads, 1) void grad_hidden_kernel(DhArgs p) {
  LP_RING
  const int tiles = p.n_ttiles * p.n_dtiles;
  const int total = tiles * p.ksplit;
  const int id = xcd_logical(blockIdx.x, total);
  const int ks = id / tiles;  // vocabulary range: tiles of one range run together
  int dt, tt;
  grouped_tile(id - ks * tiles, p.n_dtiles, p.n_ttiles, dt, tt);
  const int d0 = dt * TM, n0 = tt * TN;
  const int kb = ks * p.kper, ke = min(p.vocab, kb + p.kper);
  f32x16 acc[4][NI];
  gemm_tile<true, false>(acc, p.w + (int64_t)kb * p.ldw + d0, p.ldw, p.dim - d0, p.dl + (int64_t)n0 * p.ldl + kb,
                         p.ldl, min(TN, p.rows - n0), ke - kb, s0, s1, s2, s3);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int n = n0 + 64 * wn + 32 * ni + (lane & 31);
    if (n >= p.rows) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const int d = d0 + a_row(mi, 4 * i4, lane, wm);
        const float a[4] = {acc[mi][ni][4 * i4], acc[mi][ni][4 * i4 + 1], acc[mi][ni][4 * i4 + 2],
                            acc[mi][ni][4 * i4 + 3]};
        if (p.ksplit > 1) {
          float* q = p.part + ((int64_t)ks * p.rows + n) * p.dim + d;
          if (d + 3 < p.dim) {
            *reinterpret_cast<f32x4*>(q) = f32x4{a[0], a[1], a[2], a[3]};
          } else {
            for (int j = 0; j < 4; ++j)
              if (d + j < p.dim) q[j] = a[j];
          }
        } else if (d + 3 < p.dim) {
          *reinterpret_cast<u32x2*>(p.dh + (int64_t)n * p.ldd + d) = u32x2{pack_bf2(a[0], a[1]), pack_bf2(a[2], a[3])};
        } else {
          for (int j = 0; j < 4; ++j)
            if (d + j < p.dim) p.dh[(int64_t)n * p.ldd + d + j] = from_f<bf16>(a[j]);
        }
      }
  }
}

// dh = bf16(sum_s part[s]) in range order; four elements per thread
__global__ __launch_bounds__(kThreads) void grad_hidden_reduce_kernel(const float* __restrict__ part, int ksplit,
                                                                      int rows, int dim, bf16* __restrict__ dh,
                                                                      int64_t ldd) {
  const int64_t e = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
  const int64_t total = (int64_t)rows * dim;
  if (e >= total) return;
  const int64_t n = e / dim;
  const int d = (int)(e - n * dim);
  f32x4 s = *reinterpret_cast<const f32x4*>(part + e);
  for (int k = 1; k < ksplit; ++k) s += *reinterpret_cast<const f32x4*>(part + (int64_t)k * total + e);
  *reinterpret_cast<u32x2*>(dh + n * ldd + d) = u32x2{pack_bf2(s[0], s[1]), pack_bf2(s[2], s[3])};
}

// ---------------------------------------------------------------------------
// backward 3 (trainable head): grad_weight[v][d] += sum_n dl[n][v] h[n][d] in
// fp32, as C = dl^T . h with both operands K-strided (K = the block's rows);
// the epilogue adds the tile into the fp32 accumulator, so a call per block
// accumulates across blocks in block order.
// ---------------------------------------------------------------------------
struct DwArgs {
  const bf16* dl;   // [rows][ldl]
  int64_t ldl;
  const bf16* h;    // [rows][ldh]
  int64_t ldh;
  int rows, dim, vocab;
  int n_vtiles, n_dtiles;
  float* gw;        // [vocab][ldg]
  int64_t ldg;
};

__global__ __launch_bounds__(kGemmThreads, 1) void grad_weight_kernel(DwArgs p) {
  LP_RING
  const int total = p.n_vtiles * p.n_dtiles;
  int vt, dt;
  grouped_tile(xcd_logical(blockIdx.x, total), p.n_vtiles, p.n_dtiles, vt, dt);
  const int v0 = vt * TM, d0 = dt * TN;
  f32x16 acc[4][NI];
  gemm_tile<true, true>(acc, p.dl + v0, p.ldl, p.vocab - v0, p.h + d0, p.ldh, p.dim - d0, p.rows, s0, s1, s2,
                        s3);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int d = d0 + 64 * wn + 32 * ni + (lane & 31);
    if (d >= p.dim) continue;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int v = v0 + a_row(mi, i, lane, wm);
        if (v < p.vocab) p.gw[(int64_t)v * p.ldg + d] += acc[mi][ni][i];
      }
  }
}

// ksplit (vocabulary ranges) for grad_hidden: one work-group per CU when the
// row tiles alone do not give them, each range at least 4096 vocabulary rows
inline void grad_hidden_split(int64_t rows, int64_t dim, int64_t vocab, int& ksplit, int& kper) {
  const int64_t tiles = ((rows + TN - 1) / TN) * ((dim + TM - 1) / TM);
  int64_t k = (256 + tiles - 1) / tiles;
  k = std::min<int64_t>(k, std::max<int64_t>(1, vocab / 4096));
  k = std::max<int64_t>(1, std::min<int64_t>(k, 16));
  int64_t per = (vocab + k - 1) / k;
  per = (per + TK - 1) / TK * TK;
  ksplit = (int)((vocab + per - 1) / per);
  kper = (int)per;
}

bool ok16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace lp
}  // namespace ts

extern "C" {

int64_t ts_logprob_fwd_workspace(int64_t rows, int64_t vocab) {
  if (rows <= 0 || vocab <= 0) return 0;
  const int64_t vt = (vocab + ts::lp::BM - 1) / ts::lp::BM;
  return (3 * vt + 1) * rows * (int64_t)sizeof(float);
}

int ts_logprob_fwd(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                   const int64_t* target, int64_t rows, int64_t dim, int64_t vocab, float* logprob,
                   float* entropy, float* lse, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && vocab < (1 << 30) &&
                   dim < (1 << 20),
               "ts_logprob_fwd: bad shape rows=%lld dim=%lld vocab=%lld", (long long)rows,
               (long long)dim, (long long)vocab);
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(hidden && weight && target && logprob && lse, "ts_logprob_fwd: null pointer");
  TS_CHECK_ARG(dim % 8 == 0 && ld_hidden % 8 == 0 && ld_weight % 8 == 0 && ld_hidden >= dim &&
                   ld_weight >= dim && ok16(hidden) && ok16(weight),
               "ts_logprob_fwd: hidden/weight rows must be 16-byte aligned with dim %% 8 == 0");
  TS_CHECK_ARG(255 * ld_hidden < (1ll << 30) && 255 * ld_weight < (1ll << 30),
               "ts_logprob_fwd: leading dimensions too large for 32-bit tile offsets");
  TS_CHECK_ARG(workspace && workspace_bytes >= ts_logprob_fwd_workspace(rows, vocab),
               "ts_logprob_fwd: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
               (long long)ts_logprob_fwd_workspace(rows, vocab));
  FwdArgs a;
  a.h = (const ts::bf16*)hidden;
  a.ldh = ld_hidden;
  a.w = (const ts::bf16*)weight;
  a.ldw = ld_weight;
  a.target = target;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.n_ttiles = (int)((rows + TN - 1) / TN);
  a.n_vtiles = (int)((vocab + BM - 1) / BM);
  float* ws = (float*)workspace;
  a.part_m = ws;
  a.part_s = ws + (int64_t)a.n_vtiles * rows;
  a.part_e = ws + 2 * (int64_t)a.n_vtiles * rows;
  a.tgt = ws + 3 * (int64_t)a.n_vtiles * rows;
  TS_CHECK_ARG((int64_t)a.n_ttiles * a.n_vtiles < (1ll << 31), "ts_logprob_fwd: grid too large");
  hipStream_t s = (hipStream_t)stream;
  { ts::TimedLaunch timed_("logprob.fwd_stats_kernel", s); hipLaunchKernelGGL(fwd_stats_kernel, dim3((unsigned)(a.n_ttiles * a.n_vtiles)), dim3(kGemmThreads),
                     0, s, a); }
  int st = ts::check_launch("ts_logprob_fwd (tiles)");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.target_logit_kernel", s); hipLaunchKernelGGL(target_logit_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(kThreads),
                     0, s, a.h, a.ldh, a.w, a.ldw, target, (int)rows, (int)dim, (int)vocab, a.tgt); }
  st = ts::check_launch("ts_logprob_fwd (target logits)");
  if (st != TS_OK) return st;
  { ts::TimedLaunch timed_("logprob.combine_kernel", s); hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((rows + 63) / 64)), dim3(kThreads),
                     0, s, a.part_m, a.part_s, a.part_e, a.tgt, target, (int)rows, a.n_vtiles,
                     (int)vocab, logprob, entropy, lse); }
  return ts::check_launch("ts_logprob_fwd (combine)");
}

int ts_logprob_dlogits(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                       const int64_t* target, const float* lse, const float* entropy,
                       const float* grad_lp, const float* grad_ent, int64_t rows, int64_t dim,
                       int64_t vocab, void* dlogits, int64_t ld_dlogits, void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && vocab < (1 << 30) &&
                   dim < (1 << 20),
               "ts_logprob_dlogits: bad shape");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(hidden && weight && target && lse && grad_lp && dlogits,
               "ts_logprob_dlogits: null pointer");
  TS_CHECK_ARG(!grad_ent || entropy, "ts_logprob_dlogits: grad_ent needs the saved entropy");
  TS_CHECK_ARG(dim % 8 == 0 && ld_hidden % 8 == 0 && ld_weight % 8 == 0 && ok16(hidden) &&
                   ok16(weight) && ok16(dlogits) && ld_dlogits % 8 == 0 && ld_dlogits >= vocab,
               "ts_logprob_dlogits: alignment (16 bytes, dims %% 8) or ld_dlogits");
  TS_CHECK_ARG(255 * ld_hidden < (1ll << 30) && 255 * ld_weight < (1ll << 30),
               "ts_logprob_dlogits: leading dimensions too large for 32-bit tile offsets");
  DlArgs a;
  a.h = (const ts::bf16*)hidden;
  a.ldh = ld_hidden;
  a.w = (const ts::bf16*)weight;
  a.ldw = ld_weight;
  a.target = target;
  a.lse = lse;
  a.ent = entropy;
  a.g_lp = grad_lp;
  a.g_ent = grad_ent;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.vocab_pad = (int)((vocab + 7) / 8 * 8);
  a.n_ttiles = (int)((rows + TN - 1) / TN);
  a.n_vtiles = (int)((a.vocab_pad + BM - 1) / BM);
  a.dl = (ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  TS_CHECK_ARG(a.vocab_pad <= ld_dlogits, "ts_logprob_dlogits: ld_dlogits below padded vocab");
  { ts::TimedLaunch timed_("logprob.dlogits_kernel", (hipStream_t)stream); hipLaunchKernelGGL(dlogits_kernel, dim3((unsigned)(a.n_ttiles * a.n_vtiles)), dim3(kGemmThreads),
                     0, (hipStream_t)stream, a); }
  return ts::check_launch("ts_logprob_dlogits");
}

int64_t ts_logprob_grad_hidden_workspace(int64_t rows, int64_t dim, int64_t vocab) {
  if (rows <= 0 || dim <= 0 || vocab <= 0) return 0;
  int ksplit, kper;
  ts::lp::grad_hidden_split(rows, dim, vocab, ksplit, kper);
  return ksplit > 1 ? (int64_t)ksplit * rows * dim * (int64_t)sizeof(float) : 0;
}

int ts_logprob_grad_hidden(const void* dlogits, int64_t ld_dlogits, const void* weight, int64_t ld_weight,
                           int64_t rows, int64_t dim, int64_t vocab, void* grad_hidden, int64_t ld_grad,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && dim < (1 << 20) && vocab < (1 << 30),
               "ts_logprob_grad_hidden: bad shape");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(dlogits && weight && grad_hidden && ok16(dlogits) && ok16(weight) && ok16(grad_hidden) &&
                   ld_dlogits % 8 == 0 && ld_weight % 8 == 0 && ld_grad % 8 == 0 && dim % 8 == 0 &&
                   ld_dlogits >= (vocab + 7) / 8 * 8 && ld_weight >= dim && ld_grad >= dim,
               "ts_logprob_grad_hidden: alignment or leading dimensions");
  TS_CHECK_ARG(255 * ld_dlogits < (1ll << 30) && 31 * ld_weight < (1ll << 30),
               "ts_logprob_grad_hidden: leading dimensions too large for 32-bit tile offsets");
  DhArgs a;
  a.w = (const ts::bf16*)weight;
  a.ldw = ld_weight;
  a.dl = (const ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.n_ttiles = (int)((rows + TN - 1) / TN);
  a.n_dtiles = (int)((dim + TM - 1) / TM);
  grad_hidden_split(rows, dim, vocab, a.ksplit, a.kper);
  a.dh = (ts::bf16*)grad_hidden;
  a.ldd = ld_grad;
  a.part = (float*)workspace;
  if (a.ksplit > 1)
    TS_CHECK_ARG(workspace && workspace_bytes >= ts_logprob_grad_hidden_workspace(rows, dim, vocab) &&
                     ok16(workspace),
                 "ts_logprob_grad_hidden: workspace of %lld bytes, need %lld", (long long)workspace_bytes,
                 (long long)ts_logprob_grad_hidden_workspace(rows, dim, vocab));
  hipStream_t s = (hipStream_t)stream;
  {
    ts::TimedLaunch timed_("logprob.grad_hidden_kernel", s);
    hipLaunchKernelGGL(grad_hidden_kernel, dim3((unsigned)(a.n_ttiles * a.n_dtiles * a.ksplit)), dim3(kGemmThreads),
                       0, s, a);
  }
  int st = ts::check_launch("ts_logprob_grad_hidden");
  if (st != TS_OK || a.ksplit == 1) return st;
  const int64_t quads = rows * dim / 4;
  {
    ts::TimedLaunch timed_("logprob.grad_hidden_reduce_kernel", s);
    hipLaunchKernelGGL(grad_hidden_reduce_kernel, dim3((unsigned)((quads + kThreads - 1) / kThreads)), dim3(kThreads),
                       0, s, (const float*)workspace, a.ksplit, (int)rows, (int)dim, (ts::bf16*)grad_hidden, ld_grad);
  }
  return ts::check_launch("ts_logprob_grad_hidden (reduce)");
}

int ts_logprob_grad_weight(const void* dlogits, int64_t ld_dlogits, const void* hidden, int64_t ld_hidden,
                           int64_t rows, int64_t dim, int64_t vocab, float* grad_weight, int64_t ld_grad,
                           void* stream) {
  using namespace ts::lp;
  TS_CHECK_ARG(rows >= 0 && dim > 0 && vocab > 0 && rows < (1 << 30) && dim < (1 << 20) && vocab < (1 << 30),
               "ts_logprob_grad_weight: bad shape");
  if (rows == 0) return TS_OK;
  TS_CHECK_ARG(dlogits && hidden && grad_weight && ok16(dlogits) && ok16(hidden) && ld_dlogits % 8 == 0 &&
                   ld_hidden % 8 == 0 && dim % 8 == 0 && ld_dlogits >= vocab && ld_hidden >= dim &&
                   ld_grad >= dim,
               "ts_logprob_grad_weight: alignment or leading dimensions");
  TS_CHECK_ARG(31 * ld_dlogits < (1ll << 30) && 31 * ld_hidden < (1ll << 30),
               "ts_logprob_grad_weight: leading dimensions too large for 32-bit tile offsets");
  DwArgs a;
  a.dl = (const ts::bf16*)dlogits;
  a.ldl = ld_dlogits;
  a.h = (const ts::bf16*)hidden;
  a.ldh = ld_hidden;
  a.rows = (int)rows;
  a.dim = (int)dim;
  a.vocab = (int)vocab;
  a.n_vtiles = (int)((vocab + TM - 1) / TM);
  a.n_dtiles = (int)((dim + TN - 1) / TN);
  a.gw = grad_weight;
  a.ldg = ld_grad;
  TS_CHECK_ARG((int64_t)a.n_vtiles * a.n_dtiles < (1ll << 31), "ts_logprob_grad_weight: grid too large");
  {
    ts::TimedLaunch timed_("logprob.grad_weight_kernel", (hipStream_t)stream);
    hipLaunchKernelGGL(grad_weight_kernel, dim3((unsigned)(a.n_vtiles * a.n_dtiles)), dim3(kGemmThreads), 0,
                       (hipStream_t)stream, a);
  }
  return ts::check_launch("ts_logprob_grad_weight");
}

}  // extern "C"
