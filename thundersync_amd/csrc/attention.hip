// Forest / packed bottom-right-causal GQA attention for gfx950 (bf16, D = 128).
//
// One description (segments of query rows, runs of keys read in place, see
// include/thundersync_hip.h) drives three kernels:
//
//   fwd      query-stationary: a work-group owns a block of query rows of one
//            segment for GC query heads of one GQA group, streams the
//            segment's key runs through LDS 64 keys at a time (K and V tiles
//            shared by the GC heads), and keeps an online softmax per row.
//   dq       query-stationary like fwd, recomputing P from the saved LSE.
//   dkdv     key-stationary: a work-group owns 64 keys of one run and one KV
//            head, visits every segment that reads the run, and accumulates
//            dK/dV for all query heads of the group in registers -- no
//            atomics, fixed order, so the gradients are deterministic.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16, lane layouts pinned by the
// layout probe test):
//   fwd/dq  S^T = K Q^T  (A = K rows from LDS, B = Q^T held in registers);
//           the accumulator layout gives each lane one query column, so the
//           softmax statistics of a query live in the four lanes that share
//           (lane & 15) and P^T is already in the B-operand layout of
//           O^T += V^T P^T.  V^T (and K^T for dQ) are fed from LDS rows
//           through an 8x8 register transpose.
//   dkdv    S = Q K^T, dP = dO V^T (A from LDS rows, B = K^T/V^T held in
//           registers); dV^T += dO^T P and dK^T += Q^T dS with dO^T / Q^T
//           from LDS rows through the register transpose.
// Both sides of every contraction use the same slot permutation of the
#include "attention_impl.h"

namespace ts {
namespace attn {

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool aligned_rows(const ts_attn_rows& r) {
  return r.ptr && (r.ptr % 16 == 0) && (r.row_stride % 8 == 0) && (r.head_stride % 8 == 0) &&
         r.row_stride > 0;
}

int validate(const ts_attn_problem* p, const char* what) {
  TS_CHECK_ARG(p != nullptr, "%s: null problem", what);
  TS_CHECK_ARG(p->head_dim == D, "%s: head_dim %d unsupported (128 only)", what, p->head_dim);
  TS_CHECK_ARG(p->hq > 0 && p->hkv > 0 && p->hq % p->hkv == 0, "%s: hq %d not a multiple of hkv %d",
               what, p->hq, p->hkv);
  const int gc = heads_per_block(p->hq / p->hkv);
  TS_CHECK_ARG(p->q_block == q_block_rows(p->hq / p->hkv), "%s: q_block %d, expected %d for group %d",
               what, p->q_block, q_block_rows(p->hq / p->hkv), p->hq / p->hkv);
  TS_CHECK_ARG(p->kv_block == kv_block_keys(p->hq / p->hkv), "%s: kv_block %d, expected %d", what,
               p->kv_block, kv_block_keys(p->hq / p->hkv));
  TS_CHECK_ARG(p->n_q_work >= 0 && p->n_kv_work >= 0 && p->n_segs >= 0 && p->n_runs >= 0,
               "%s: negative table size", what);
  TS_CHECK_ARG(p->n_q_long >= 0 && p->n_q_long <= p->n_q_work && p->n_kv_long >= 0 &&
               p->n_kv_long <= p->n_kv_work, "%s: long-item counts outside the work lists", what);
  TS_CHECK_ARG(p->n_q_work == 0 || (p->q_work && p->segs && p->seg_spans && p->runs),
               "%s: null table", what);
  TS_CHECK_ARG((int64_t)p->n_q_work * (p->hq / gc) < (1ll << 31) && (int64_t)p->n_kv_work * p->hkv < (1ll << 31),
               "%s: work list too long", what);
  return TS_OK;
}

}  // namespace attn
}  // namespace ts

extern "C" {

int ts_attn_heads_per_block(int group) { return group > 0 ? ts::attn::heads_per_block(group) : 0; }

int ts_attn_kv_block(int group) { return group > 0 ? ts::attn::kv_block_keys(group) : 0; }
int ts_attn_q_block(int group) { return group > 0 ? ts::attn::q_block_rows(group) : 0; }

int ts_attn_fwd(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out, float* lse,
                int64_t lse_ld, void* stream) {
  using namespace ts::attn;
  int st = validate(problem, "ts_attn_fwd");
  if (st != TS_OK) return st;
  const ts_attn_problem& P = *problem;
  if (P.n_q_work == 0) return TS_OK;
  TS_CHECK_ARG(aligned_rows(q) && aligned_rows(out), "ts_attn_fwd: q/out must be 16-byte aligned "
               "with strides that are multiples of 8 elements");
  TS_CHECK_ARG(lse && lse_ld >= P.q_rows, "ts_attn_fwd: lse null or lse_ld %lld < rows %lld",
               (long long)lse_ld, (long long)P.q_rows);
  return launch_fwd(P, q, out, lse, lse_ld, (hipStream_t)stream);
}

int ts_attn_bwd(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out, ts_attn_rows dout,
                const float* lse, int64_t lse_ld, float* rowstats, ts_attn_rows dq, void* stream) {
  using namespace ts::attn;
  int st = validate(problem, "ts_attn_bwd");
  if (st != TS_OK) return st;
  const ts_attn_problem& P = *problem;
  if (P.n_q_work == 0 && P.n_kv_work == 0) return TS_OK;
  TS_CHECK_ARG(aligned_rows(q) && aligned_rows(out) && aligned_rows(dout) && aligned_rows(dq),
               "ts_attn_bwd: q/out/dout/dq must be 16-byte aligned with strides that are "
               "multiples of 8 elements");
  TS_CHECK_ARG(q.row_stride < (1ll << 25) && dout.row_stride < (1ll << 25),
               "ts_attn_bwd: q/dout row strides must be below 2^25 elements");
  TS_CHECK_ARG(lse && rowstats && lse_ld >= P.q_rows, "ts_attn_bwd: lse/rowstats null or lse_ld too small");
  TS_CHECK_ARG(P.n_kv_work == 0 || (P.kv_work && P.run_visits), "ts_attn_bwd: null kv tables");
  hipStream_t s = (hipStream_t)stream;
  st = launch_delta(P, out, dout, lse, rowstats, lse_ld, s);
  if (st != TS_OK) return st;
  if (P.n_q_work > 0) {
    st = launch_dq(P, q, dout, rowstats, lse_ld, dq, s);
    if (st != TS_OK) return st;
  }
  if (P.n_kv_work > 0) st = launch_dkdv(P, q, dout, rowstats, lse_ld, s);
  return st;
}

}  // extern "C"

