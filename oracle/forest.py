"""Forest / plan / pack-layout metadata oracle (CPU, pure Python).

Restates, step for step, the reference's integer metadata builders:

* ``build_forest`` and ``_longest_common_prefix``
  (src/thundersync/engine/segments.py:243-346): a radix trie over
  ``(token, scored)`` keys per group, groups in sorted order, nodes emitted in
  pre-order, children in sorted key order (:336);
* ``compile_plan`` (engine/plan.py:166-340): DFS pre-order layout
  (:173-178), per-node token/position/node arrays, ``subtree_end``
  (:226-241), ``key_ranges`` (:248-256), scoring slots (:266-297), logical
  view (:304-319);
* ``visibility_mask`` (engine/plan.py:343-362);
* the pack layout's cumulative lengths and input order
  (engine/streaming.py:1613-1698).

Pinned by golden vectors the reference itself produced
(tests/golden/forest_metadata.json, written by
tests/golden/make_forest_golden.py) and by the invariants
tests/test_forest_metadata.py checks: a trajectory's physical path
reproduces its tokens and scoring mask; ``kv <= q < subtree_end[kv]`` equals
the dense visibility mask; every logical scored token maps to a slot whose
source is its predecessor.
"""

from __future__ import annotations

from dataclasses import dataclass, field


@dataclass(frozen=True)
class Segment:
    tokens: tuple
    kind: str
    scored: bool


@dataclass
class Trajectory:
    segments: list
    group_id: int = 0
    traj_id: int = 0

    def keyed(self):
        return [(t, s.scored) for s in self.segments for t in s.tokens]

    @property
    def tokens(self):
        return [t for s in self.segments for t in s.tokens]

    @property
    def scored_mask(self):
        return [s.scored for s in self.segments for _ in s.tokens]


@dataclass
class Node:
    tokens: list
    scored: list
    parent: int | None
    depth: int
    trajectories: list
    children: list = field(default_factory=list)
    group_id: int = 0


@dataclass
class Forest:
    nodes: list
    roots: list
    trajectories: list
    leaf_of: dict

    def path_to_root(self, node):
        path = []
        cur = node
        while cur is not None:
            path.append(cur)
            cur = self.nodes[cur].parent
        path.reverse()
        return path


def longest_common_prefix(seqs):
    """segments.py:243-264 (binary search over slice equality)."""
    if not seqs:
        return 0
    hi = min(len(s) for s in seqs)
    if len(seqs) == 1:
        return hi
    lo = 0
    while lo < hi:
        mid = (lo + hi + 1) // 2
        ref = seqs[0][:mid]
        if all(s[:mid] == ref for s in seqs[1:]):
            lo = mid
        else:
            hi = mid - 1
    return lo


def build_forest(trajectories):
    """segments.py:280-346."""
    nodes, roots, leaf_of = [], [], {}
    by_group = {}
    for t in trajectories:
        by_group.setdefault(t.group_id, []).append(t)
    for group_id, members in sorted(by_group.items()):
        keyed = {t.traj_id: t.keyed() for t in members}

        def emit(traj_ids, offset, parent, depth):
            suffixes = [keyed[i][offset:] for i in traj_ids]
            share = longest_common_prefix(suffixes)
            if share == 0 and parent is not None:
                raise AssertionError("zero-length non-root node: partition is wrong")
            head = suffixes[0][:share] if share else []
            idx = len(nodes)
            nodes.append(Node([k[0] for k in head], [k[1] for k in head], parent, depth,
                              list(traj_ids), group_id=group_id))
            if parent is None:
                roots.append(idx)
            else:
                nodes[parent].children.append(idx)
            nxt = offset + share
            ongoing = {}
            for i in traj_ids:
                if len(keyed[i]) == nxt:
                    leaf_of[i] = idx
                else:
                    ongoing.setdefault(keyed[i][nxt], []).append(i)
            for _, group in sorted(ongoing.items()):
                emit(group, nxt, idx, depth + 1)

        emit([t.traj_id for t in members], 0, None, 0)
    return Forest(nodes, roots, list(trajectories), leaf_of)


def compile_plan(forest):
    """plan.py:166-340, as plain Python lists."""
    nodes = forest.nodes
    order = []
    stack = list(reversed(forest.roots))
    while stack:
        n = stack.pop()
        order.append(n)
        stack.extend(reversed(nodes[n].children))

    start, end, pos_offset = {}, {}, {}
    token_ids, position_ids, node_of = [], [], []
    cursor = 0
    for n in order:
        node = nodes[n]
        parent = node.parent
        pos_offset[n] = 0 if parent is None else pos_offset[parent] + len(nodes[parent].tokens)
        ln = len(node.tokens)
        start[n] = cursor
        cursor += ln
        end[n] = cursor
        token_ids.extend(node.tokens)
        position_ids.extend(range(pos_offset[n], pos_offset[n] + ln))
        node_of.extend([n] * ln)

    subtree_node_end = {}
    for n in reversed(order):
        subtree_node_end[n] = max([end[n], *(subtree_node_end[c] for c in nodes[n].children)])
    subtree_end = []
    for n in order:
        subtree_end.extend([subtree_node_end[n]] * (end[n] - start[n]))

    key_ranges = [[] for _ in nodes]
    for n in order:
        parent = nodes[n].parent
        inherited = [] if parent is None else key_ranges[parent][:-1] + [(start[parent], end[parent])]
        key_ranges[n] = [(s, e) for s, e in inherited if e > s] + [(start[n], end[n])]

    score_src, score_tgt, score_pos = [], [], []
    slot_start, slot_count = {}, {}
    n_slots = 0
    for n in order:
        node = nodes[n]
        parent = node.parent
        slot_start[n] = n_slots
        slot_count[n] = 0
        if not node.tokens:
            continue
        sc = list(node.scored)
        if parent is None:
            sc[0] = False
        js = [j for j, s in enumerate(sc) if s]
        if not js:
            continue
        for j in js:
            p = j + start[n]
            src = p - 1
            if parent is not None and j == 0:
                src = end[parent] - 1
            score_src.append(src)
            score_pos.append(p)
            score_tgt.append(node.tokens[j])
        slot_count[n] = len(js)
        n_slots += len(js)

    logical_to_slot, logical_traj = [], []
    for traj in forest.trajectories:
        leaf = forest.leaf_of[traj.traj_id]
        total = 0
        for n in forest.path_to_root(leaf):
            c = slot_count.get(n, 0)
            if c:
                logical_to_slot.extend(range(slot_start[n], slot_start[n] + c))
                total += c
        logical_traj.extend([traj.traj_id] * total)

    return {
        "token_ids": token_ids,
        "position_ids": position_ids,
        "node_of": node_of,
        "node_start": [start[n] for n in range(len(nodes))],
        "node_end": [end[n] for n in range(len(nodes))],
        "node_parent": [-1 if nodes[n].parent is None else nodes[n].parent for n in range(len(nodes))],
        "node_depth": [nodes[n].depth for n in range(len(nodes))],
        "subtree_end": subtree_end,
        "score_src": score_src,
        "score_tgt": score_tgt,
        "score_pos": score_pos,
        "logical_to_slot": logical_to_slot,
        "logical_traj": logical_traj,
        "key_ranges": [[list(r) for r in kr] for kr in key_ranges],
    }


def visibility_mask(plan):
    """plan.py:343-362 as a list of lists of bools."""
    p = len(plan["token_ids"])
    mask = [[False] * p for _ in range(p)]
    for n in range(len(plan["node_start"])):
        s, e = plan["node_start"][n], plan["node_end"][n]
        if s == e:
            continue
        spans = plan["key_ranges"][n]
        for ks, ke in spans[:-1]:
            for q in range(s, e):
                for k in range(ks, ke):
                    mask[q][k] = True
        for q in range(s, e):
            for k in range(s, q + 1):
                mask[q][k] = True
    return mask


def pack_cumulative(lengths, prefixes):
    """engine/streaming.py:1693-1694: int32 [0, *accumulate(...)]."""
    cu_l, cu_p = [0], [0]
    for n in lengths:
        cu_l.append(cu_l[-1] + n)
    for n in prefixes:
        cu_p.append(cu_p[-1] + n)
    return cu_l, cu_p


def pack_input_order(ancestor_counts):
    """engine/streaming.py:1636-1650: (segment, chunk) per input position,
    grouped by segment, LAST segment first."""
    out = []
    for s in reversed(range(len(ancestor_counts))):
        out.extend((s, c) for c in range(ancestor_counts[s]))
    return out
