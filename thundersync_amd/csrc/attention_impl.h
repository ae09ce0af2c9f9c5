// Device helpers and host launchers shared by the attention translation units
// (attention.hip: entry points; attention_fwd.hip, attention_dq.hip,
// attention_dkdv.hip: kernels).  The kernels are compiled in separate units
// so each can take its own code-generation flags.
#pragma once
#include <type_traits>

#include "common.h"
#include "timing.h"
#include "../../include/thundersync_hip.h"

namespace ts {
namespace attn {


constexpr int D = 128;
constexpr int BK = 64;          // keys per tile (fwd / dq) and per dkdv block
constexpr int kThreads = 256;   // 4 waves
constexpr int PITCH = D + 8;    // LDS row pitch in elements (272 bytes)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ float neg_inf() { return -__builtin_huge_valf(); }

__device__ __forceinline__ u32x4 ld16(const bf16* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(bf16* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }

// Head dims the kernels take: a multiple of 32 up to 256.  128 runs the
// tuned one-wave-per-head kernels (GQA groups that are a multiple of 4); every
// other head dim, and groups that are not a multiple of 4, run the
// register-staged kernels below, templated on the head dim HD.
__host__ __device__ constexpr bool head_dim_supported(int hd) {
  return hd == 32 || hd == 64 || hd == 96 || hd == 128 || hd == 192 || hd == 256;
}

// LDS row pitch (elements) of the register-staged kernels' tiles: 16 bytes of
// padding per row
template <int HD> constexpr int pitch_of() { return HD + 8; }

// A 64 x HD tile of K or V rows moved global -> registers -> LDS by 256
// threads; HD / 8 consecutive threads read one row.
template <int HD>
struct Tile {
  u32x4 v[HD / 32];
};

template <int HD>
__device__ __forceinline__ void tile_load(Tile<HD>& t, const bf16* base, int64_t row_stride, int nvalid,
                                          int tid) {
  constexpr int CH = HD / 8;
#pragma unroll
  for (int it = 0; it < HD / 32; ++it) {
    const int idx = it * kThreads + tid;
    const int row = idx / CH, chunk = idx % CH;
    if (row < nvalid)
      t.v[it] = ld16(base + (int64_t)row * row_stride + chunk * 8);
    else
      t.v[it] = u32x4{0u, 0u, 0u, 0u};
  }
}

template <int HD>
__device__ __forceinline__ void tile_store(const Tile<HD>& t, bf16* lds, int tid) {
  constexpr int CH = HD / 8;
#pragma unroll
  for (int it = 0; it < HD / 32; ++it) {
    const int idx = it * kThreads + tid;
    st16(lds + (idx / CH) * pitch_of<HD>() + (idx % CH) * 8, t.v[it]);
  }
}

// One 64-key K tile and V tile into LDS (all threads; the barriers order the
// stores after every wave's reads of the previous tiles and the reads after
// the stores).  Up to a head dim of 128 both tiles are in flight at once;
// above it they go one after the other, halving the staging registers.
template <int HD>
__device__ __forceinline__ void stage_kv(bf16* sk, bf16* sv, const bf16* kp, int64_t k_stride, const bf16* vp,
                                         int64_t v_stride, int nvalid, int tid) {
  if constexpr (HD <= 128) {
    Tile<HD> tk, tv;
    tile_load(tk, kp, k_stride, nvalid, tid);
    tile_load(tv, vp, v_stride, nvalid, tid);
    __syncthreads();
    tile_store(tk, sk, tid);
    tile_store(tv, sv, tid);
  } else {
    Tile<HD> t;
    tile_load(t, kp, k_stride, nvalid, tid);
    __syncthreads();
    tile_store(t, sk, tid);
    tile_load(t, vp, v_stride, nvalid, tid);
    tile_store(t, sv, tid);
  }
  __syncthreads();
}

// rows [0, 32) x HD of a per-head query-row tensor -> LDS (256 threads)
template <int HD = D>
__device__ __forceinline__ void rows32_to_lds(bf16* lds, const bf16* base, int64_t row_stride,
                                              int nvalid, int tid) {
  constexpr int CH = HD / 8;
#pragma unroll
  for (int idx = tid; idx < 32 * CH; idx += kThreads) {
    const int row = idx / CH, chunk = idx % CH;
    u32x4 v = u32x4{0u, 0u, 0u, 0u};
    if (row < nvalid) v = ld16(base + (int64_t)row * row_stride + chunk * 8);
    st16(lds + row * pitch_of<HD>() + chunk * 8, v);
  }
}

// the row of slot j for lane group g: 4g + (j & 3) + 16 (j >> 2)
__device__ __forceinline__ void slot_rows(int g, int base, int rows[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) rows[j] = base + 4 * g + (j & 3) + 16 * (j >> 2);
}

// eight floats as eight T values (an operand container; see mma16)
template <typename T> __device__ __forceinline__ bf16x8 pack8(const float* x) {
  u32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = pack2<T>(x[2 * i], x[2 * i + 1]);
  return as_bf16x8(r);
}

// Load a wave's 16 NQB query rows x HD as B operands of S^T = K Q^T:
// reg[qb][ks] = row (16 qb + (lane & 15)), columns 32 ks + 8 (lane >> 4) .. +7.
template <int NQB, int HD = D>
__device__ __forceinline__ void load_rows_b(bf16x8 (&reg)[NQB][HD / 32], const bf16* base, int64_t row_stride,
                                            int nvalid, int lane) {
#pragma unroll
  for (int qb = 0; qb < NQB; ++qb) {
    const int row = 16 * qb + (lane & 15);
#pragma unroll
    for (int ks = 0; ks < HD / 32; ++ks) {
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (row < nvalid) v = ld16(base + (int64_t)row * row_stride + 32 * ks + 8 * (lane >> 4));
      reg[qb][ks] = as_bf16x8(v);
    }
  }
}

// S^T tile (64 keys x 32 rows) = K_lds Q^T: s[kb][qb] lane holds keys
// 16 kb + 4 (lane >> 4) + i, row 16 qb + (lane & 15).
template <typename E, int HD = D>
__device__ __forceinline__ void tile_scores(f32x4 s[4][2], const bf16* sk, const bf16x8 qreg[2][HD / 32],
                                            int lane) {
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    s[kb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    s[kb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < HD / 32; ++ks) {
      const bf16x8 a = as_bf16x8(ld16(sk + (16 * kb + (lane & 15)) * pitch_of<HD>() + 32 * ks + 8 * (lane >> 4)));
      s[kb][0] = mma16<E>(a, qreg[0][ks], s[kb][0]);
      s[kb][1] = mma16<E>(a, qreg[1][ks], s[kb][1]);
    }
  }
}

// The grid is one-dimensional over (work item, head chunk) pairs.  Work lists
// are sorted longest first.  The first n_long items run item-major (every
// head's longest items start before any short ones, so none is left for the
// tail of the launch); the remaining items run head-major, all XCDs streaming
// the same head's rows through the shared last-level cache.  Work-groups are
// dispatched round-robin over the 8 XCDs (linear id b runs on XCD b % 8);
// within every full window of 64 head-major ids XCD c receives 8 consecutive
// items of one head, neighbours in the cost-sorted list that read the same
// rows and share its L2.  Returns the work item; `y` receives the head chunk.
__device__ __forceinline__ int task_of(int n_items, int n_long, int& y) {
  const int t = (int)blockIdx.x;
  const int gy = (int)gridDim.x / n_items;
  if (t < n_long * gy) {
    const int item = t / gy;
    y = t - item * gy;
    return item;
  }
  const int n_rest = n_items - n_long;
  const int b = t - n_long * gy;
  const int base = b & ~63;
  int u = b;
  if (base + 64 <= n_rest * gy) {
    const int r = b & 63;
    u = base + ((r & 7) << 3) + (r >> 3);
  }
  y = u / n_rest;
  return n_long + (u - y * n_rest);
}


// ---------------------------------------------------------------------------
// 256-byte-row LDS tiles (buffer DMA + transposed reads)
// ---------------------------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr int kTile32 = 32 * D;              // elements of one 32-row tile (256-byte rows)
// Q tile + dO tile + 32 (lse2, delta) pairs in a 1 KB slot: the statistics
// DMA is issued by all 64 lanes (lanes 16.. with an out-of-range offset write
// zeros into the rest of the slot), so it needs no lane branch
constexpr int kStage32 = 2 * kTile32 + 512;

__device__ __forceinline__ u32x2 tr_read(const bf16* p) {
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)p);
  u32x2 r;
  __builtin_memcpy(&r, &v, 8);
  return r;
}

// A transposed operand of the register-staged kernels from a padded LDS tile
// (row pitch HD + 8 elements) by two ds_read_b64_tr_b16: the 16 x 32 A
// operand X^T[16 mb .. 16 mb + 15][row0 + slot rows], slot j <-> row
// row0 + 16 (j >> 2) + 4 g4 + (j & 3) (the slot order of slot_rows).  Lane
// (g4, j16) addresses row row0 + 4 g4 + j16 / 4 and columns
// 16 mb + 4 (j16 & 3) .. + 3, and receives X[row0 + 4 g4 + t][16 mb + j16],
// t = 0..3, then the same from 16 rows further.
template <int HD>
__device__ __forceinline__ bf16x8 tr_frag(const bf16* lds, int row0, int mb, int lane) {
  const int g4 = lane >> 4, j16 = lane & 15;
  const bf16* p = lds + (row0 + 4 * g4 + (j16 >> 2)) * pitch_of<HD>() + 16 * mb + 4 * (j16 & 3);
  const u32x2 a = tr_read(p), b = tr_read(p + 16 * pitch_of<HD>());
  return as_bf16x8(u32x4{a[0], a[1], b[0], b[1]});
}

// A key run's position in its visit list with the visited segment's fields
// cached, so that advancing by a row block reads no table unless it moves to
// the next visit.
struct VisitCursor {
  int vi;          // visit index; >= nvisit at the end
  int r0;          // first row of the block (segment-local)
  int q_len;       // rows of the visited segment
  int off;         // its kv_len - q_len
  int kpos;        // position of the run's first key in the segment's key order
  int64_t q_row0;  // its first row in the packed Q / dO / statistics
};

// ---------------------------------------------------------------------------
// dS workspace: the backward route that stores dS once and forms dQ = dS K
// from it instead of recomputing S and dP in the dQ kernel.
//
// The dK/dV kernels compute dS = P (dP - delta) for every visible (row, key)
// pair, rounded to the element type for their dK product; on this route they
// also store it.  Unit of storage: a block of 32 query rows x 16 keys (512
// elements) of one (segment, span) pair of one query head.  The blocks of a
// pair form its rectangle: row block rb (segment rows 32 rb .. 32 rb + 31)
// holds the run's 16-key blocks 0 .. n(rb) - 1, the prefix that some row of
// it below q_len sees, row block after row block (invisible blocks take no
// space).  A head's rectangles sit at the offsets of the span and visit
// tables; heads follow one another.
//
// Inside a block, row r and key k: slot s = 8 ((r >> 2) & 3) + 4 (r >> 4) +
// (r & 3) (so lane (g4, j16) of a dK/dV wave, which holds rows 16 qb + 4 g4 + i
// of key j16, owns slots 8 g4 .. 8 g4 + 7), element 32 k + 8 (c ^ ((k >> 1) &
// 2)) + (s & 7) with c = s >> 3: 64-byte key rows of four 16-byte chunks,
// the chunks of keys 4..7 and 12..15 swapped in pairs so that the dQ
// kernel's transposed LDS reads of keys 4 g4 + t (lanes g4 = 0, 1 in one
// pass) touch distinct banks.
// ---------------------------------------------------------------------------
constexpr int kDsBlock = 512;  // elements of a 32-row x 16-key block

struct DsArgs {
  const int64_t* span;   // per seg_spans entry: element offset of its rectangle within a head
  const int64_t* visit;  // per run_visits entry: that of the span it visits
  int64_t head;          // elements per head
  uint64_t ptr;          // device address of the workspace (hq * head elements)
  const int32_t* dq_work;  // the dQ pass's 64-row work list (groups of 4 at head dim 128), or null
  int32_t n_dq_work, n_dq_long;
};

// One (segment, span) rectangle: row r of the segment sees run key j iff
// j <= d + r (d = kv_len - q_len - kpos); nkb 16-key blocks; q_len rows.
struct DsRect {
  int d;
  int nkb;
  int q_len;
};

__host__ __device__ inline int64_t imin64(int64_t a, int64_t b) { return a < b ? a : b; }
__host__ __device__ inline int64_t imax64(int64_t a, int64_t b) { return a > b ? a : b; }

// key blocks stored for row block rb: those holding a key that one of its
// rows below q_len sees
__host__ __device__ inline int ds_blocks_in(const DsRect& R, int rb) {
  const int64_t maxrow = imin64(32 * (int64_t)rb + 31, R.q_len - 1);
  const int64_t last = R.d + maxrow;  // the last run key that row sees
  return last < 0 ? 0 : (int)imin64(R.nkb, last / 16 + 1);
}

// blocks stored before row block rb (rb below the last row block + 1): the
// earlier row blocks are whole (32 rows below q_len), row block t holding
// clamp(2 t + c, 0, nkb) blocks with c = floor((d + 31) / 16) + 1; summed in
// closed form over the zero, linear and saturated stretches of t.  Floor
// divisions by powers of two are arithmetic shifts (no branches).
__host__ __device__ inline int64_t ds_blocks_before(const DsRect& R, int rb) {
  const int64_t c = (((int64_t)R.d + 31) >> 4) + 1, n = R.nkb;
  const int64_t t0 = imax64(0, ((-c) >> 1) + 1);  // first t with 2 t + c > 0
  const int64_t t1 = imax64(0, -((c - n) >> 1));  // first t with 2 t + c >= n
  const int64_t b = imin64(rb, t1), a = imin64(t0, b);
  return (b - a) * (a + b - 1 + c) + n * imax64(0, rb - t1);
}

// blocks of the whole rectangle
__host__ __device__ inline int64_t ds_rect_blocks(const DsRect& R) {
  const int nrb = (R.q_len + 31) >> 5;
  return nrb == 0 ? 0 : ds_blocks_before(R, nrb - 1) + ds_blocks_in(R, nrb - 1);
}

// 16 bytes to global memory through a global-address-space pointer: a
// global store (a generic pointer makes it a FLAT store, which also counts
// on the LDS counter and so turns every later LDS wait into a full drain),
// non-temporal (the dS stream is read back once, by another kernel: its
// lines should not displace the Q/dO and K/V lines the kernels reuse)
__device__ __forceinline__ void global_st16(bf16* p, u32x4 v) {
  __builtin_nontemporal_store(v, (__attribute__((address_space(1))) u32x4*)(p));
}

// byte offset of lane (g4, j16)'s 16-byte store of its dS slots in a block
__device__ __forceinline__ int ds_store_offset(int lane) {
  const int g4 = lane >> 4, j16 = lane & 15;
  return 64 * j16 + 16 * (g4 ^ ((j16 >> 1) & 2));
}




constexpr int kKV64 = BK * D;  // elements of one 64-key tile

struct TileCursor {
  int sp;          // span index; == nspan at the end
  int kt0;         // first run-local key of the tile
  int kpos;        // position of the span's first key in the segment's key order
  int len;         // keys of the span's run
  const bf16* kt;  // K row kt0 of the KV head (advanced with kt0 within a span)
  const bf16* vt;  // V row kt0 likewise
  int k_rs, v_rs;  // the run's row strides (elements, below 2^24)
};

// cache span tc.sp's reference and run fields, at the span's first key of KV
// head hk (tc.sp < nspan)
__device__ __forceinline__ void enter_span(const ts_attn_problem& P, const ts_attn_segment& seg, int hk,
                                           TileCursor& tc) {
  const ts_attn_ref ref = load_uniform(P.seg_spans, seg.span0 + tc.sp);
  const ts_attn_run run = load_uniform(P.runs, ref.index);
  tc.kpos = ref.kpos;
  tc.len = run.len;
  tc.k_rs = (int)run.k_row_stride;
  tc.v_rs = (int)run.v_row_stride;
  tc.kt = (const bf16*)run.k + (int64_t)hk * run.k_head_stride;
  tc.vt = (const bf16*)run.v + (int64_t)hk * run.v_head_stride;
}

// `tc` itself if some row up to `last` (segment-local) can see its tile, else
// the next such tile in the segment's key order; sp == nspan when none is
// left.  Spans are in key order, so once a tile starts past the last visible
// key so do all later ones.  Tables are read only on entering a span.
template <int KT = BK>
__device__ __forceinline__ TileCursor settle_kv_tile(const ts_attn_problem& P, const ts_attn_segment& seg, int hk,
                                                     int last, TileCursor tc) {
  const int off = seg.kv_len - seg.q_len;
  while (tc.sp < seg.nspan) {
    if (tc.kt0 >= tc.len) {
      if (++tc.sp < seg.nspan) enter_span(P, seg, hk, tc);
      tc.kt0 = 0;
      continue;
    }
    if (tc.kpos + tc.kt0 > off + last) tc.sp = seg.nspan;
    break;
  }
  return tc;
}

// the visible tile after `tc`: the K / V pointers advance by KT rows within a
// span (no table reads, no 64-bit products)
template <int KT = BK>
__device__ __forceinline__ TileCursor next_kv_tile(const ts_attn_problem& P, const ts_attn_segment& seg, int hk,
                                                   int last, TileCursor tc) {
  tc.kt0 += KT;
  tc.kt += KT * tc.k_rs;
  tc.vt += KT * tc.v_rs;
  return settle_kv_tile<KT>(P, seg, hk, last, tc);
}

// the first visible tile of a segment
template <int KT = BK>
__device__ __forceinline__ TileCursor first_kv_tile(const ts_attn_problem& P, const ts_attn_segment& seg, int hk,
                                                    int last) {
  TileCursor tc{0, 0, 0, 0, nullptr, nullptr, 0, 0};
  if (seg.nspan > 0) enter_span(P, seg, hk, tc);
  return settle_kv_tile<KT>(P, seg, hk, last, tc);
}

// Row swizzle of the 256-byte-row LDS tiles: 16-byte chunk c of row r sits at
// slot c ^ tile_swizzle(r & 15).  Measured on the MI355X with a read-rate probe
// (reads issued back to back, no other work): a ds_read_b128 is serviced in
// four passes of 16 lanes, a pass being the lanes with equal (lane >> 5) and
// equal ((lane >> 4) ^ (lane >> 2) ^ (lane >> 3)) & 1; a ds_read_b64_tr_b16 in
// two passes of 32 lanes.  A tile's 16-row fragment reads (lane (g4, j16):
// row j16, chunk 4 ks + g4) and its transposed reads (row 4 g4 + j16 / 4,
// chunks 2 mb, 2 mb + 1) are conflict-free when every pass covers 16 distinct
// slots, which holds for s(r) = r ^ (r & 1 ? 12 : 0) (4.2 clk per b128 and
// 2.2 clk per transposed read per CU, against 4.2 and 4.1 for s(r) = r).
__device__ __forceinline__ int tile_swizzle(int r) { return r ^ ((r & 1) ? 12 : 0); }

// DMA of the cursor's K/V tile of KT keys into swizzled LDS tiles (rows of
// HD elements, chunk c of row r at slot c ^ tile_swizzle(r & 15)).  The WAVES
// waves of a work-group (4 or 8) each issue instructions t = wave + WAVES u;
// instruction t fills rows RPI t .. RPI t + RPI - 1 (RPI = 4 at HD 128, 2 at
// 256): lane l the row RPI t + l / (HD / 8), slot l % (HD / 8) with logical
// chunk (l % (HD / 8)) ^ tile_swizzle(row).  Rows past the run arrive as
// zeros.
template <int WAVES = 4, int HD = D, int KT = BK>
__device__ __forceinline__ void issue_kv_tile(int wave, int lane, const TileCursor& tc, bf16* sk, bf16* sv) {
  static_assert(WAVES == 4 || WAVES == 8, "a tile is 16 or 32 instructions");
  static_assert(HD == 128 || HD == 256, "the swizzle needs 16 or 32 chunks per row");
  constexpr int CH = HD / 8, RPI = 64 / CH, NI = KT / RPI;
  static_assert(NI % WAVES == 0, "every wave issues the same number of instructions");
  const int nvalid = min(KT, tc.len - tc.kt0);
  const rsrc_t rk = make_rsrc(tc.kt, (uint32_t)(nvalid * tc.k_rs * 2));
  const rsrc_t rv = make_rsrc(tc.vt, (uint32_t)(nvalid * tc.v_rs * 2));
  if constexpr (HD == 128) {
    // rows 4 t + g4: the swizzle of row 4 (t + WAVES u) + g4 is that of row 4 t + g4
    const int g4 = lane >> 4, j16 = lane & 15;
    const int dma_row = 4 * wave + g4;
    const int dma_chunk = (j16 ^ tile_swizzle((4 * wave + g4) & 15)) << 3;
    const int ko = (dma_row * tc.k_rs + dma_chunk) * 2;
    const int vo = (dma_row * tc.v_rs + dma_chunk) * 2;
    const int kstep = 4 * WAVES * tc.k_rs * 2, vstep = 4 * WAVES * tc.v_rs * 2;
#pragma unroll
    for (int u = 0; u < NI / WAVES; ++u) {
      buffer_dma16(rk, sk + (wave + WAVES * u) * 512, ko + u * kstep);
      buffer_dma16(rv, sv + (wave + WAVES * u) * 512, vo + u * vstep);
    }
  } else {
#pragma unroll
    for (int u = 0; u < NI / WAVES; ++u) {
      const int t = wave + WAVES * u;
      const int row = RPI * t + lane / CH;
      const int chunk = ((lane % CH) ^ tile_swizzle(row & 15)) << 3;
      buffer_dma16(rk, sk + t * 512, (row * tc.k_rs + chunk) * 2);
      buffer_dma16(rv, sv + t * 512, (row * tc.v_rs + chunk) * 2);
    }
  }
}

// per-lane LDS offsets (elements) into a swizzled tile of HD-element rows:
// ro[ks]: row j16, logical chunk 4 ks + g4 (A-operand row reads of 16 rows);
// to[mb]: row 4 g4 + j16 / 4, columns 16 mb + 4 (j16 & 3) .. + 3 (the
// addresses of a ds_read_b64_tr_b16 that yields X[4 g4 + t][16 mb + j16]).
// The swizzle permutes chunks within aligned groups of 16, so at head dim 256
// the offsets of k-step ks + 4 and column block mb + 8 are those of ks and mb
// plus 128 elements: only the first four and eight are kept (the rest fold
// into the reads' immediate offsets).
template <int HD = D>
__device__ __forceinline__ void swizzled_offsets(int lane, int ro[4], int to[8]) {
  const int g4 = lane >> 4, j16 = lane & 15;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ro[ks] = j16 * HD + (((4 * ks + g4) ^ tile_swizzle(j16)) << 3);
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int r = 4 * g4 + (j16 >> 2);
    const int col = 16 * mb + 4 * (j16 & 3);
    to[mb] = r * HD + (((col >> 3) ^ tile_swizzle(r)) << 3) + (col & 7);
  }
}
// the offsets of k-step ks and column block mb
__device__ __forceinline__ int ro_of(const int ro[4], int ks) { return ro[ks & 3] + 128 * (ks >> 2); }
__device__ __forceinline__ int to_of(const int to[8], int mb) { return to[mb & 7] + 128 * (mb >> 3); }


// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
inline int heads_per_block(int group) {
  if (group % 4 == 0) return 4;
  if (group % 2 == 0) return 2;
  return 1;
}

// query rows per forward / dQ work item: 32 per query head of the work-group
inline int q_block_rows(int group) { return 32 * 4 / heads_per_block(group); }

// keys per dK/dV work-group: 48 for the one-wave-per-head kernel (GQA groups
// that are a multiple of 4 below head dim 256: its 192 dK/dV accumulators and
// 48 S/dP values fill the 256 AGPRs), else 64 (at head dim 256 the two waves
// of 32 keys of dkdv256_kernel, every group)
inline int kv_block_keys(int group, int head_dim) { return group % 4 == 0 && head_dim != 256 ? 48 : BK; }

// launchers (one per kernel family); each returns a TS_* status
int launch_fwd(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows out, float* lse, int64_t lse_ld,
               hipStream_t s);
int launch_delta(const ts_attn_problem& P, ts_attn_rows out, ts_attn_rows dout, const float* lse,
                 float* rowstats, int64_t lse_ld, hipStream_t s);
int launch_dq(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout, const float* rowstats,
              int64_t lse_ld, ts_attn_rows dq, hipStream_t s);
// `ds` null: dK/dV only; else the kernels also store dS into the workspace
// (only where ds_route holds)
int launch_dkdv(const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout, const float* rowstats,
                int64_t lse_ld, const DsArgs* ds, hipStream_t s);
// the one-wave-per-head dK/dV kernel (groups that are a multiple of 4, head
// dim 128; attention_dkdv_wave.hip), storing dS when DS
template <typename E, bool DS>
void launch_dkdv_wave(dim3 grid, const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout,
                      const float* rowstats, int64_t lse_ld, const DsArgs& S, hipStream_t s);
// the head-dim-256 dK/dV kernel with 32 keys per wave (64-key work items;
// attention_dkdv256.hip), storing dS when DS
template <typename E, bool DS>
void launch_dkdv256(dim3 grid, const ts_attn_problem& P, ts_attn_rows q, ts_attn_rows dout,
                    const float* rowstats, int64_t lse_ld, const DsArgs& S, hipStream_t s);
// dQ = scale dS K from the workspace the dK/dV launch filled
int launch_dq_ds(const ts_attn_problem& P, const DsArgs& ds, ts_attn_rows dq, hipStream_t s);

// the dS route: head dims 128 and 256 (the DMA-staged dK/dV kernels), every
// GQA group size
inline bool ds_route(int head_dim, int /*group*/) { return head_dim == 128 || head_dim == 256; }

}  // namespace attn
}  // namespace ts
