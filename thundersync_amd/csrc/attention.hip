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
#include <vector>

#include "attention_impl.h"

// the host mirrors (thundersync_amd/_abi.py) assume these sizes
static_assert(sizeof(ts_attn_problem) == 112 && sizeof(ts_attn_rows) == 24, "ts_attn ABI layout");

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
  TS_CHECK_ARG(head_dim_supported(p->head_dim), "%s: head_dim %d unsupported (32, 64, 96, 128, 192 or 256)", what,
               p->head_dim);
  TS_CHECK_ARG(p->dtype == kBF16 || p->dtype == kF16, "%s: dtype %d unsupported (bf16 or fp16)", what, p->dtype);
  TS_CHECK_ARG(p->hq > 0 && p->hkv > 0 && p->hq % p->hkv == 0, "%s: hq %d not a multiple of hkv %d",
               what, p->hq, p->hkv);
  const int gc = heads_per_block(p->hq / p->hkv);
  TS_CHECK_ARG(p->q_block == q_block_rows(p->hq / p->hkv), "%s: q_block %d, expected %d for group %d",
               what, p->q_block, q_block_rows(p->hq / p->hkv), p->hq / p->hkv);
  // head dim 256 also takes 48-key items (the key-split kernel: few work items)
  TS_CHECK_ARG(p->kv_block == kv_block_keys(p->hq / p->hkv, p->head_dim) || (p->head_dim == 256 && p->kv_block == 48),
               "%s: kv_block %d, expected %d", what, p->kv_block, kv_block_keys(p->hq / p->hkv, p->head_dim));
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

// delta, then dQ and dK/dV: recomputing S and dP in the dQ kernel (`ds`
// null), or storing dS in the dK/dV kernels and forming dQ = dS K from it
int backward(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out, ts_attn_rows dout,
             const float* lse, int64_t lse_ld, float* rowstats, ts_attn_rows dq, const DsArgs* ds,
             const char* what, void* stream) {
  int st = validate(problem, what);
  if (st != TS_OK) return st;
  const ts_attn_problem& P = *problem;
  if (P.n_q_work == 0 && P.n_kv_work == 0) return TS_OK;
  TS_CHECK_ARG(aligned_rows(q) && aligned_rows(out) && aligned_rows(dout) && aligned_rows(dq),
               "%s: q/out/dout/dq must be 16-byte aligned with strides that are "
               "multiples of 8 elements", what);
  TS_CHECK_ARG(q.row_stride < (1ll << 25) && dout.row_stride < (1ll << 25),
               "%s: q/dout row strides must be below 2^25 elements", what);
  TS_CHECK_ARG(lse && rowstats && lse_ld >= P.q_rows, "%s: lse/rowstats null or lse_ld too small", what);
  TS_CHECK_ARG(P.n_kv_work == 0 || (P.kv_work && P.run_visits), "%s: null kv tables", what);
  // every row block reads dS that the dK/dV items store: with no dK/dV items
  // (no visited run) there is nothing to read and the recompute runs
  if (P.n_kv_work == 0) ds = nullptr;
  hipStream_t s = (hipStream_t)stream;
  st = launch_delta(P, out, dout, lse, rowstats, lse_ld, s);
  if (st != TS_OK) return st;
  if (ds) {
    st = launch_dkdv(P, q, dout, rowstats, lse_ld, ds, s);
    if (st == TS_OK && P.n_q_work > 0) st = launch_dq_ds(P, *ds, dq, s);
    return st;
  }
  if (P.n_q_work > 0) {
    st = launch_dq(P, q, dout, rowstats, lse_ld, dq, s);
    if (st != TS_OK) return st;
  }
  if (P.n_kv_work > 0) st = launch_dkdv(P, q, dout, rowstats, lse_ld, nullptr, s);
  return st;
}

}  // namespace attn
}  // namespace ts

extern "C" {

int ts_attn_heads_per_block(int group) { return group > 0 ? ts::attn::heads_per_block(group) : 0; }

int ts_attn_kv_block(int group, int head_dim) { return group > 0 ? ts::attn::kv_block_keys(group, head_dim) : 0; }
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
  return ts::attn::backward(problem, q, out, dout, lse, lse_ld, rowstats, dq, nullptr, "ts_attn_bwd", stream);
}

int ts_attn_ds_route(int head_dim, int group) { return group > 0 && ts::attn::ds_route(head_dim, group) ? 1 : 0; }

int ts_attn_ds_layout(const ts_attn_segment* segs, int32_t n_segs, const ts_attn_ref* seg_spans, int64_t n_spans,
                      const int32_t* run_len, int32_t n_runs, const ts_attn_ref* run_visits,
                      const int32_t* visit0, const int32_t* nvisit, int64_t n_visits, int64_t* span_ds,
                      int64_t* visit_ds, int64_t* ds_head) {
  using namespace ts::attn;
  const char* what = "ts_attn_ds_layout";
  TS_CHECK_ARG(n_segs >= 0 && n_spans >= 0 && n_runs >= 0 && n_visits >= 0 && ds_head, "%s: bad sizes", what);
  TS_CHECK_ARG((n_segs == 0 || segs) && (n_spans == 0 || (seg_spans && span_ds)) &&
                   (n_runs == 0 || (run_len && visit0 && nvisit)) && (n_visits == 0 || (run_visits && visit_ds)),
               "%s: null table", what);
  int64_t total = 0;
  for (int32_t s = 0; s < n_segs; ++s) {
    const ts_attn_segment& g = segs[s];
    TS_CHECK_ARG(g.q_len >= 0 && g.span0 >= 0 && g.nspan >= 0 && (int64_t)g.span0 + g.nspan <= n_spans,
                 "%s: segment %d spans [%d, %d) outside the %lld spans", what, s, g.span0, g.span0 + g.nspan,
                 (long long)n_spans);
    for (int32_t i = 0; i < g.nspan; ++i) {
      const ts_attn_ref& r = seg_spans[g.span0 + i];
      TS_CHECK_ARG(r.index >= 0 && r.index < n_runs && run_len[r.index] > 0, "%s: segment %d span %d names run %d",
                   what, s, i, r.index);
      span_ds[g.span0 + i] = total;
      const DsRect R{g.kv_len - g.q_len - r.kpos, (run_len[r.index] + 15) >> 4, g.q_len};
      total += ds_rect_blocks(R) * kDsBlock;
    }
  }
  for (int32_t r = 0; r < n_runs; ++r) {
    TS_CHECK_ARG(visit0[r] >= 0 && nvisit[r] >= 0 && (int64_t)visit0[r] + nvisit[r] <= n_visits,
                 "%s: run %d visits outside the %lld visits", what, r, (long long)n_visits);
    for (int32_t i = 0; i < nvisit[r]; ++i) {
      const ts_attn_ref& v = run_visits[visit0[r] + i];
      TS_CHECK_ARG(v.index >= 0 && v.index < n_segs, "%s: run %d visit %d names segment %d", what, r, i, v.index);
      const ts_attn_segment& g = segs[v.index];
      int32_t j = 0;
      while (j < g.nspan && !(seg_spans[g.span0 + j].index == r && seg_spans[g.span0 + j].kpos == v.kpos)) ++j;
      TS_CHECK_ARG(j < g.nspan, "%s: run %d visit %d is not a span of segment %d", what, r, i, v.index);
      visit_ds[visit0[r] + i] = span_ds[g.span0 + j];
    }
  }
  *ds_head = total;
  return TS_OK;
}

int ts_attn_bwd_ds(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out, ts_attn_rows dout,
                   const float* lse, int64_t lse_ld, float* rowstats, ts_attn_rows dq, const int64_t* span_ds,
                   const int64_t* visit_ds, int64_t ds_head, void* ds, int64_t ds_bytes, const int32_t* dq_work,
                   int32_t n_dq_work, int32_t n_dq_long, void* stream) {
  using namespace ts::attn;
  const char* what = "ts_attn_bwd_ds";
  TS_CHECK_ARG(problem != nullptr, "%s: null problem", what);
  if (problem->hkv <= 0 || problem->hq % problem->hkv || !ds_route(problem->head_dim, problem->hq / problem->hkv))
    return backward(problem, q, out, dout, lse, lse_ld, rowstats, dq, nullptr, what, stream);
  TS_CHECK_ARG(ds_head >= 0 && problem->hq > 0 && ds_bytes / 2 >= kDsBlock &&
                   (ds_bytes / 2 - kDsBlock) / problem->hq >= ds_head,
               "%s: workspace of %lld bytes below (%d heads x %lld + 512) elements", what, (long long)ds_bytes,
               problem->hq, (long long)ds_head);
  TS_CHECK_ARG((problem->n_q_work == 0 && problem->n_kv_work == 0) ||
                   (ds && (uint64_t)ds % 16 == 0 && span_ds && visit_ds),
               "%s: null or unaligned workspace or tables", what);
  TS_CHECK_ARG(!dq_work || (n_dq_work >= 0 && n_dq_long >= 0 && n_dq_long <= n_dq_work &&
                             (int64_t)n_dq_work * problem->hq < (1ll << 31)),
               "%s: dQ work list counts", what);
  TS_CHECK_ARG(!dq_work || (problem->head_dim == 128 && (problem->hq / problem->hkv) % 4 == 0),
               "%s: a dQ work list is for GQA groups that are a multiple of 4 at head dim 128", what);
  const DsArgs args{span_ds, visit_ds, ds_head, (uint64_t)ds, dq_work, n_dq_work, n_dq_long};
  return backward(problem, q, out, dout, lse, lse_ld, rowstats, dq, &args, what, stream);
}

int ts_attn_check_tables(const ts_attn_problem* problem, const ts_attn_segment* segs,
                         const ts_attn_ref* seg_spans, int64_t n_spans, const ts_attn_run* runs,
                         const ts_attn_ref* run_visits, int64_t n_visits, const int32_t* q_work,
                         const int32_t* kv_work) {
  using namespace ts::attn;
  const char* what = "ts_attn_check_tables";
  int st = validate(problem, what);
  if (st != TS_OK) return st;
  const ts_attn_problem& P = *problem;
  TS_CHECK_ARG(n_spans >= 0 && n_visits >= 0 && (P.n_segs == 0 || (segs && (n_spans == 0 || seg_spans))) &&
                   (P.n_runs == 0 || runs) && (n_visits == 0 || run_visits) && (P.n_q_work == 0 || q_work) &&
                   (P.n_kv_work == 0 || kv_work),
               "%s: null host table", what);
  // runs: lengths, addressing, visit ranges
  for (int32_t r = 0; r < P.n_runs; ++r) {
    const ts_attn_run& u = runs[r];
    TS_CHECK_ARG(u.len > 0, "%s: run %d has length %d", what, r, u.len);
    TS_CHECK_ARG(u.k && u.v && u.k % 16 == 0 && u.v % 16 == 0 && u.k_row_stride > 0 && u.v_row_stride > 0 &&
                     u.k_row_stride % 8 == 0 && u.v_row_stride % 8 == 0 && u.k_head_stride % 8 == 0 &&
                     u.v_head_stride % 8 == 0 && u.k_row_stride < (1 << 24) && u.v_row_stride < (1 << 24),
                 "%s: run %d K/V need 16-byte aligned rows, strides multiples of 8 below 2^24", what, r);
    TS_CHECK_ARG((!u.dk || (u.dk % 16 == 0 && u.dk_row_stride % 8 == 0 && u.dk_head_stride % 8 == 0)) &&
                     (!u.dv || (u.dv % 16 == 0 && u.dv_row_stride % 8 == 0 && u.dv_head_stride % 8 == 0)),
                 "%s: run %d dK/dV need 16-byte aligned rows and strides multiples of 8", what, r);
    TS_CHECK_ARG(u.visit0 >= 0 && u.nvisit >= 0 && (int64_t)u.visit0 + u.nvisit <= n_visits,
                 "%s: run %d visits [%d, %d) outside the %lld visits", what, r, u.visit0, u.visit0 + u.nvisit,
                 (long long)n_visits);
  }
  // segments and their spans: each span list tiles the segment's keys in order
  int64_t q_blocks = 0;
  for (int32_t s = 0; s < P.n_segs; ++s) {
    const ts_attn_segment& g = segs[s];
    TS_CHECK_ARG(g.q_row0 >= 0 && g.q_len >= 0 && g.q_row0 + g.q_len <= P.q_rows,
                 "%s: segment %d rows [%lld, %lld) outside [0, %lld)", what, s, (long long)g.q_row0,
                 (long long)(g.q_row0 + g.q_len), (long long)P.q_rows);
    TS_CHECK_ARG(g.q_len == 0 || g.kv_len >= g.q_len, "%s: segment %d has %d rows over %d keys", what, s,
                 g.q_len, g.kv_len);
    TS_CHECK_ARG(g.span0 >= 0 && g.nspan >= 0 && (int64_t)g.span0 + g.nspan <= n_spans,
                 "%s: segment %d spans [%d, %d) outside the %lld spans", what, s, g.span0, g.span0 + g.nspan,
                 (long long)n_spans);
    int64_t pos = 0;
    for (int32_t i = 0; i < g.nspan; ++i) {
      const ts_attn_ref& r = seg_spans[g.span0 + i];
      TS_CHECK_ARG(r.index >= 0 && r.index < P.n_runs, "%s: segment %d span %d names run %d of %d", what, s, i,
                   r.index, P.n_runs);
      TS_CHECK_ARG(r.kpos == pos, "%s: segment %d span %d at key %d, expected %lld", what, s, i, r.kpos,
                   (long long)pos);
      pos += runs[r.index].len;
    }
    TS_CHECK_ARG(pos == g.kv_len, "%s: segment %d spans cover %lld keys, kv_len %d", what, s, (long long)pos,
                 g.kv_len);
    q_blocks += (g.q_len + P.q_block - 1) / P.q_block;
  }
  // visits that match the segments' spans one to one
  int64_t visits = 0, kv_blocks = 0;
  std::vector<char> span_seen(n_spans, 0);
  for (int32_t r = 0; r < P.n_runs; ++r) {
    const ts_attn_run& u = runs[r];
    for (int32_t i = 0; i < u.nvisit; ++i) {
      const ts_attn_ref& v = run_visits[u.visit0 + i];
      TS_CHECK_ARG(v.index >= 0 && v.index < P.n_segs, "%s: run %d visit %d names segment %d of %d", what, r,
                   i, v.index, P.n_segs);
      const ts_attn_segment& g = segs[v.index];
      int32_t j = 0;
      while (j < g.nspan && !(seg_spans[g.span0 + j].index == r && seg_spans[g.span0 + j].kpos == v.kpos)) ++j;
      TS_CHECK_ARG(j < g.nspan, "%s: run %d visit %d (segment %d, key %d) is not a span of that segment", what,
                   r, i, v.index, v.kpos);
      TS_CHECK_ARG(!span_seen[g.span0 + j], "%s: run %d visit %d repeats segment %d span %d", what, r, i, v.index,
                   j);
      span_seen[g.span0 + j] = 1;
    }
    visits += u.nvisit;
    if (u.nvisit > 0) kv_blocks += (u.len + P.kv_block - 1) / P.kv_block;
  }
  int64_t spans_used = 0;
  for (int32_t s = 0; s < P.n_segs; ++s) spans_used += segs[s].nspan;
  TS_CHECK_ARG(visits == spans_used, "%s: %lld visits for %lld spans", what, (long long)visits,
               (long long)spans_used);
  // work lists: every row block and every visited run's key block exactly once
  TS_CHECK_ARG(P.n_q_work == q_blocks && P.n_kv_work == kv_blocks,
               "%s: %d forward items for %lld row blocks, %d dK/dV items for %lld key blocks", what, P.n_q_work,
               (long long)q_blocks, P.n_kv_work, (long long)kv_blocks);
  std::vector<int64_t> first_q(P.n_segs + 1, 0), first_k(P.n_runs + 1, 0);
  for (int32_t s = 0; s < P.n_segs; ++s) first_q[s + 1] = first_q[s] + (segs[s].q_len + P.q_block - 1) / P.q_block;
  for (int32_t r = 0; r < P.n_runs; ++r)
    first_k[r + 1] = first_k[r] + (runs[r].nvisit > 0 ? (runs[r].len + P.kv_block - 1) / P.kv_block : 0);
  std::vector<char> seen_q(q_blocks, 0), seen_k(kv_blocks, 0);
  for (int32_t i = 0; i < P.n_q_work; ++i) {
    const int32_t s = q_work[2 * i], q0 = q_work[2 * i + 1];
    TS_CHECK_ARG(s >= 0 && s < P.n_segs && q0 >= 0 && q0 < segs[s].q_len && q0 % P.q_block == 0,
                 "%s: forward item %d (segment %d, row %d) is not a row block", what, i, s, q0);
    char& once = seen_q[first_q[s] + q0 / P.q_block];
    TS_CHECK_ARG(!once, "%s: forward item %d repeats segment %d row %d", what, i, s, q0);
    once = 1;
  }
  for (int32_t i = 0; i < P.n_kv_work; ++i) {
    const int32_t r = kv_work[2 * i], k0 = kv_work[2 * i + 1];
    TS_CHECK_ARG(r >= 0 && r < P.n_runs && runs[r].nvisit > 0 && k0 >= 0 && k0 < runs[r].len &&
                     k0 % P.kv_block == 0,
                 "%s: dK/dV item %d (run %d, key %d) is not a key block of a visited run", what, i, r, k0);
    char& once = seen_k[first_k[r] + k0 / P.kv_block];
    TS_CHECK_ARG(!once, "%s: dK/dV item %d repeats run %d key %d", what, i, r, k0);
    once = 1;
  }
  return TS_OK;
}

}  // extern "C"

