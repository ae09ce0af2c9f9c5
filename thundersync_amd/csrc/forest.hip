// Segment forest and execution plan: the integer metadata every kernel call
// consumes, built on the host in one pass over flat key arrays.
//
// Reference: engine/segments.py:243-346 (build_forest) and
// engine/plan.py:166-340 (compile_plan).  The conventions that make the output
// bit-exact with the reference are kept:
//
// * a key is 2 * token + scored, so ascending keys are ascending
//   (token, scored) pairs (segments.py:336 sorts children by that pair);
// * groups in ascending group id, a group's trajectories in input order;
//   a node holds the longest key prefix all of its trajectories share from its
//   offset; trajectories that end there make it their leaf, the rest split by
//   their next key into children, created in ascending key order; nodes are
//   numbered in creation order, which is pre-order;
// * the plan lays nodes out in the pre-order the caller passes; a root's first
//   token is never scored; a node's first scored token is predicted by its
//   parent's last physical token, end[parent] - 1 (-1 below a zero-length
//   root, as plan.py:281-290 computes it); slots are handed out node by node
//   in layout order, and the logical view walks each trajectory root to leaf
//   (plan.py:304-319).
//
// Host code only: there is no device code in this file.
#include <algorithm>
#include <utility>
#include <vector>

#include "common.h"
#include "../../include/thundersync_hip.h"

namespace {

struct Work {
  std::vector<int64_t> ids;  // trajectory indices, input order
  int64_t offset, parent, depth;
};

}  // namespace

extern "C" {

int ts_forest_build(int64_t n_traj, const int64_t* group_id, const int64_t* key_offsets, const int64_t* keys,
                    int64_t max_nodes, int64_t* n_nodes, int64_t* node_parent, int64_t* node_depth,
                    int64_t* node_group, int64_t* node_src, int64_t* node_offset, int64_t* node_len,
                    int64_t* leaf_of) {
  TS_CHECK_ARG(n_traj >= 0 && n_nodes && (n_traj == 0 || (group_id && key_offsets && leaf_of)),
               "ts_forest_build: null argument (n_traj=%lld)", (long long)n_traj);
  TS_CHECK_ARG(max_nodes >= 2 * n_traj, "ts_forest_build: max_nodes %lld < 2 * n_traj %lld",
               (long long)max_nodes, (long long)(2 * n_traj));
  for (int64_t i = 0; i < n_traj; ++i)
    TS_CHECK_ARG(key_offsets[i + 1] > key_offsets[i], "ts_forest_build: trajectory %lld is empty or offsets fall",
                 (long long)i);
  // groups ascending, members in input order
  std::vector<int64_t> by_group(n_traj);
  for (int64_t i = 0; i < n_traj; ++i) by_group[i] = i;
  std::stable_sort(by_group.begin(), by_group.end(),
                   [&](int64_t a, int64_t b) { return group_id[a] < group_id[b]; });
  auto key = [&](int64_t t, int64_t j) { return keys[key_offsets[t] + j]; };
  auto len = [&](int64_t t) { return key_offsets[t + 1] - key_offsets[t]; };

  int64_t nn = 0;
  std::vector<Work> stack;
  std::vector<std::pair<int64_t, int64_t>> next;  // (next key, trajectory)
  for (int64_t g0 = 0; g0 < n_traj;) {
    int64_t g1 = g0;
    while (g1 < n_traj && group_id[by_group[g1]] == group_id[by_group[g0]]) ++g1;
    stack.push_back(Work{std::vector<int64_t>(by_group.begin() + g0, by_group.begin() + g1), 0, -1, 0});
    while (!stack.empty()) {
      Work w = std::move(stack.back());
      stack.pop_back();
      const int64_t first = w.ids[0];
      int64_t share = len(first) - w.offset;
      for (int64_t t : w.ids) share = std::min(share, len(t) - w.offset);
      for (size_t m = 1; m < w.ids.size() && share > 0; ++m) {
        const int64_t t = w.ids[m];
        int64_t j = 0;
        while (j < share && key(t, w.offset + j) == key(first, w.offset + j)) ++j;
        share = j;
      }
      share = std::max<int64_t>(share, 0);
      TS_CHECK_ARG(share > 0 || w.parent < 0, "ts_forest_build: zero-length non-root node");
      TS_CHECK_ARG(nn < max_nodes, "ts_forest_build: more than %lld nodes", (long long)max_nodes);
      const int64_t idx = nn++;
      node_parent[idx] = w.parent;
      node_depth[idx] = w.depth;
      node_group[idx] = group_id[first];
      node_src[idx] = first;
      node_offset[idx] = w.offset;
      node_len[idx] = share;
      const int64_t at = w.offset + share;
      next.clear();
      for (int64_t t : w.ids) {
        if (len(t) == at) leaf_of[t] = idx;
        else next.emplace_back(key(t, at), t);
      }
      // stable by key keeps input order inside a branch
      std::stable_sort(next.begin(), next.end(),
                       [](const std::pair<int64_t, int64_t>& a, const std::pair<int64_t, int64_t>& b) {
                         return a.first < b.first;
                       });
      // branches pushed in descending key order, so the smallest pops first
      size_t hi = next.size();
      while (hi > 0) {
        size_t lo = hi - 1;
        while (lo > 0 && next[lo - 1].first == next[hi - 1].first) --lo;
        Work child{{}, at, idx, w.depth + 1};
        child.ids.reserve(hi - lo);
        for (size_t m = lo; m < hi; ++m) child.ids.push_back(next[m].second);
        stack.push_back(std::move(child));
        hi = lo;
      }
    }
    g0 = g1;
  }
  *n_nodes = nn;
  return TS_OK;
}

int ts_plan_compile(int64_t n_nodes, const int64_t* node_parent, const int64_t* order, const int64_t* node_len,
                    const int64_t* node_key_offsets, const int64_t* keys, int64_t n_traj, const int64_t* traj_leaf,
                    const int64_t* traj_id, int64_t max_logical, int64_t* token_ids, int64_t* position_ids,
                    int64_t* node_of, int64_t* node_start, int64_t* node_end, int64_t* subtree_end,
                    int64_t* score_src, int64_t* score_tgt, int64_t* score_pos, int64_t* n_scored,
                    int64_t* logical_to_slot, int64_t* logical_traj, int64_t* n_logical) {
  TS_CHECK_ARG(n_nodes >= 0 && n_traj >= 0 && n_scored && n_logical, "ts_plan_compile: null argument");
  std::vector<int64_t> pos0(n_nodes, 0), sub_end(n_nodes, 0), slot_start(n_nodes, 0), slot_count(n_nodes, 0);
  std::vector<char> seen(n_nodes, 0);
  for (int64_t r = 0; r < n_nodes; ++r) {
    const int64_t n = order[r];
    TS_CHECK_ARG(n >= 0 && n < n_nodes && !seen[n], "ts_plan_compile: order is not a permutation (at %lld)",
                 (long long)r);
    seen[n] = 1;
    const int64_t p = node_parent[n];
    TS_CHECK_ARG(p < n_nodes && (p < 0 || seen[p]), "ts_plan_compile: node %lld comes before its parent",
                 (long long)n);
    TS_CHECK_ARG(node_len[n] >= 0, "ts_plan_compile: node %lld has a negative length", (long long)n);
  }
  // layout: DFS pre-order, positions continue the parent's
  int64_t cursor = 0;
  for (int64_t r = 0; r < n_nodes; ++r) {
    const int64_t n = order[r], p = node_parent[n];
    pos0[n] = p < 0 ? 0 : pos0[p] + node_len[p];
    node_start[n] = cursor;
    for (int64_t j = 0; j < node_len[n]; ++j) {
      token_ids[cursor + j] = keys[node_key_offsets[n] + j] >> 1;
      position_ids[cursor + j] = pos0[n] + j;
      node_of[cursor + j] = n;
    }
    cursor += node_len[n];
    node_end[n] = cursor;
    sub_end[n] = cursor;
  }
  // a subtree ends where its last descendant ends (children follow parents in pre-order)
  for (int64_t r = n_nodes - 1; r >= 0; --r) {
    const int64_t n = order[r], p = node_parent[n];
    if (p >= 0) sub_end[p] = std::max(sub_end[p], sub_end[n]);
  }
  for (int64_t r = 0; r < n_nodes; ++r) {
    const int64_t n = order[r];
    for (int64_t j = node_start[n]; j < node_end[n]; ++j) subtree_end[j] = sub_end[n];
  }
  // scored targets, slot by slot in layout order
  int64_t slots = 0;
  for (int64_t r = 0; r < n_nodes; ++r) {
    const int64_t n = order[r], p = node_parent[n];
    slot_start[n] = slots;
    for (int64_t j = 0; j < node_len[n]; ++j) {
      const int64_t k = keys[node_key_offsets[n] + j];
      if (!(k & 1) || (p < 0 && j == 0)) continue;
      score_pos[slots] = node_start[n] + j;
      score_src[slots] = (j == 0) ? node_end[p] - 1 : node_start[n] + j - 1;
      score_tgt[slots] = k >> 1;
      ++slots;
    }
    slot_count[n] = slots - slot_start[n];
  }
  *n_scored = slots;
  // logical view: each trajectory root to leaf, in input order
  int64_t nl = 0;
  std::vector<int64_t> path;
  for (int64_t t = 0; t < n_traj; ++t) {
    path.clear();
    for (int64_t n = traj_leaf[t]; n >= 0; n = node_parent[n]) {
      TS_CHECK_ARG(n < n_nodes && path.size() <= (size_t)n_nodes, "ts_plan_compile: trajectory %lld has a bad path",
                   (long long)t);
      path.push_back(n);
    }
    for (auto it = path.rbegin(); it != path.rend(); ++it) {
      const int64_t c = slot_count[*it];
      TS_CHECK_ARG(nl + c <= max_logical, "ts_plan_compile: more than %lld logical slots", (long long)max_logical);
      for (int64_t s = 0; s < c; ++s) {
        logical_to_slot[nl + s] = slot_start[*it] + s;
        logical_traj[nl + s] = traj_id[t];
      }
      nl += c;
    }
  }
  *n_logical = nl;
  return TS_OK;
}

}  // extern "C"
