"""Segment forest and execution plan: the integer metadata the kernels consume.

Same API and bit-identical outputs as the reference's
``engine/segments.py`` (``Segment``, ``Trajectory``, ``build_forest``) and
``engine/plan.py`` (``ExecutionPlan``, ``compile_plan``,
``visibility_mask``), built differently: the radix trie is grown with an
explicit work stack and numpy mismatch scans instead of recursion and binary
search over slices, and the plan arrays are assembled with numpy over whole
nodes.  The conventions that make the output bit-exact are kept:

* groups in ascending ``group_id``; a node's children in ascending
  ``(token, scored)`` order of their first key (segments.py:336);
* nodes numbered in pre-order; layout in DFS pre-order from ``roots``
  (plan.py:173-178);
* a root's first token is never scored, and a node's first scored token is
  predicted by its parent's last token -- ``end[parent] - 1``, which is
  ``-1`` below a zero-length grouping root, exactly as the reference
  computes it (plan.py:281-290);
* slots handed out node by node in layout order; the logical view walks
  each trajectory root-to-leaf in input order (plan.py:304-319).

Checked against golden vectors the reference produced
(tests/golden/forest_metadata.json).
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence
from dataclasses import dataclass, field
from enum import Enum

import numpy as np
import torch


class SegmentKind(str, Enum):
    PROMPT = "prompt"
    ACTION = "action"
    OBSERVATION = "observation"


@dataclass(frozen=True)
class Segment:
    """A run of tokens with one provenance and one scoring decision."""

    tokens: tuple[int, ...]
    kind: SegmentKind
    scored: bool

    def __post_init__(self) -> None:
        if not self.tokens:
            raise ValueError("a segment must contain at least one token")

    def __len__(self) -> int:
        return len(self.tokens)

    @classmethod
    def prompt(cls, tokens: Iterable[int], *, scored: bool = False) -> "Segment":
        return cls(tuple(tokens), SegmentKind.PROMPT, scored)

    @classmethod
    def action(cls, tokens: Iterable[int], *, scored: bool = True) -> "Segment":
        return cls(tuple(tokens), SegmentKind.ACTION, scored)

    @classmethod
    def observation(cls, tokens: Iterable[int], *, scored: bool = False) -> "Segment":
        return cls(tuple(tokens), SegmentKind.OBSERVATION, scored)


@dataclass
class Trajectory:
    segments: list[Segment]
    group_id: int = 0
    traj_id: int = 0

    def __post_init__(self) -> None:
        if not self.segments:
            raise ValueError("a trajectory must contain at least one segment")

    @property
    def tokens(self) -> list[int]:
        return [t for s in self.segments for t in s.tokens]

    @property
    def scored_mask(self) -> list[bool]:
        return [s.scored for s in self.segments for _ in s.tokens]

    @property
    def n_tokens(self) -> int:
        return sum(len(s) for s in self.segments)

    def keys(self) -> np.ndarray:
        """``(token, scored)`` packed as ``2 * token + scored`` (order-preserving)."""
        parts = [np.asarray(s.tokens, dtype=np.int64) * 2 + int(s.scored) for s in self.segments]
        return np.concatenate(parts) if parts else np.zeros(0, np.int64)

    def keyed(self) -> list[tuple[int, bool]]:
        return [(t, s.scored) for s in self.segments for t in s.tokens]


@dataclass
class ForestNode:
    tokens: list[int]
    scored: list[bool]
    parent: int | None
    depth: int
    trajectories: list[int]
    children: list[int] = field(default_factory=list)
    group_id: int = 0

    @property
    def n_tokens(self) -> int:
        return len(self.tokens)

    @property
    def multiplicity(self) -> int:
        return len(self.trajectories)


@dataclass
class SegmentForest:
    nodes: list[ForestNode]
    roots: list[int]
    trajectories: list[Trajectory]
    leaf_of: dict[int, int]

    @property
    def physical_tokens(self) -> int:
        return sum(n.n_tokens for n in self.nodes)

    @property
    def logical_tokens(self) -> int:
        return sum(t.n_tokens for t in self.trajectories)

    def path_to_root(self, node: int) -> list[int]:
        path = []
        cur: int | None = node
        while cur is not None:
            path.append(cur)
            cur = self.nodes[cur].parent
        return path[::-1]


def _shared_prefix(keys: list[np.ndarray], offset: int) -> int:
    """Length of the prefix all ``keys[i][offset:]`` agree on."""
    first = keys[0]
    limit = min(len(k) for k in keys) - offset
    share = limit
    for k in keys[1:]:
        if share == 0:
            break
        diff = np.flatnonzero(first[offset : offset + share] != k[offset : offset + share])
        if diff.size:
            share = int(diff[0])
    return max(share, 0)


def build_forest(trajectories: Sequence[Trajectory]) -> SegmentForest:
    """Compress trajectories into the exact shared forest (segments.py:280-346 semantics)."""
    nodes: list[ForestNode] = []
    roots: list[int] = []
    leaf_of: dict[int, int] = {}
    groups: dict[int, list[Trajectory]] = {}
    for t in trajectories:
        groups.setdefault(t.group_id, []).append(t)
    for group_id in sorted(groups):
        members = groups[group_id]
        keys = {t.traj_id: t.keys() for t in members}
        # work stack of (trajectory ids, offset, parent, depth); popped in pre-order
        stack = [([t.traj_id for t in members], 0, None, 0)]
        while stack:
            ids, offset, parent, depth = stack.pop()
            share = _shared_prefix([keys[i] for i in ids], offset)
            if share == 0 and parent is not None:
                raise AssertionError("zero-length non-root node: partition is wrong")
            head = keys[ids[0]][offset : offset + share]
            idx = len(nodes)
            nodes.append(ForestNode(
                tokens=(head >> 1).tolist(), scored=(head & 1).astype(bool).tolist(), parent=parent,
                depth=depth, trajectories=list(ids), group_id=group_id,
            ))
            if parent is None:
                roots.append(idx)
            else:
                nodes[parent].children.append(idx)
            nxt = offset + share
            branches: dict[int, list[int]] = {}
            for i in ids:
                if len(keys[i]) == nxt:
                    leaf_of[i] = idx
                else:
                    branches.setdefault(int(keys[i][nxt]), []).append(i)
            for key in sorted(branches, reverse=True):
                stack.append((branches[key], nxt, idx, depth + 1))
    return SegmentForest(nodes, roots, list(trajectories), leaf_of)


@dataclass
class ExecutionPlan:
    """A forest laid out for execution (fields of engine/plan.py:41-73)."""

    token_ids: torch.Tensor
    position_ids: torch.Tensor
    node_of: torch.Tensor
    node_start: torch.Tensor
    node_end: torch.Tensor
    node_parent: torch.Tensor
    node_depth: torch.Tensor
    subtree_end: torch.Tensor
    score_src: torch.Tensor
    score_tgt: torch.Tensor
    score_pos: torch.Tensor
    logical_to_slot: torch.Tensor
    logical_traj: torch.Tensor
    key_ranges: list[list[tuple[int, int]]]
    forest: SegmentForest

    @property
    def n_physical(self) -> int:
        return int(self.token_ids.shape[0])

    @property
    def n_scored(self) -> int:
        return int(self.score_src.shape[0])

    @property
    def n_nodes(self) -> int:
        return int(self.node_start.shape[0])

    @property
    def is_two_level(self) -> bool:
        return int(self.node_depth.max().item()) <= 1 if self.n_nodes else True

    def physical_path(self, traj_id: int) -> list[int]:
        out: list[int] = []
        for n in self.forest.path_to_root(self.forest.leaf_of[traj_id]):
            out.extend(range(int(self.node_start[n]), int(self.node_end[n])))
        return out

    def to(self, device, *, non_blocking: bool = False) -> "ExecutionPlan":
        target = torch.device(device)
        if self.token_ids.device == target:
            return self
        moved = {
            name: getattr(self, name).to(target, non_blocking=non_blocking)
            for name in ("token_ids", "position_ids", "node_of", "node_start", "node_end", "node_parent",
                         "node_depth", "subtree_end", "score_src", "score_tgt", "score_pos",
                         "logical_to_slot", "logical_traj")
        }
        return ExecutionPlan(**moved, key_ranges=self.key_ranges, forest=self.forest)


def _preorder(forest: SegmentForest) -> list[int]:
    order, stack = [], list(reversed(forest.roots))
    while stack:
        n = stack.pop()
        order.append(n)
        stack.extend(reversed(forest.nodes[n].children))
    return order


def compile_plan(forest: SegmentForest, device: torch.device | str = "cpu") -> ExecutionPlan:
    """Lay the forest out in DFS pre-order and derive every index from it."""
    nodes = forest.nodes
    order = _preorder(forest)
    nn = len(nodes)
    lengths = np.array([len(n.tokens) for n in nodes], np.int64)
    start = np.zeros(nn, np.int64)
    end = np.zeros(nn, np.int64)
    pos0 = np.zeros(nn, np.int64)
    cursor = 0
    for n in order:
        p = nodes[n].parent
        pos0[n] = 0 if p is None else pos0[p] + lengths[p]
        start[n] = cursor
        cursor += lengths[n]
        end[n] = cursor
    ordered = [n for n in order if lengths[n]]
    counts = lengths[ordered] if ordered else np.zeros(0, np.int64)
    tokens = np.concatenate([np.asarray(nodes[n].tokens, np.int64) for n in ordered]) if ordered else np.zeros(0, np.int64)
    node_of = np.repeat(np.asarray(ordered, np.int64), counts)
    node_pos0 = np.repeat(pos0[ordered], counts) if ordered else np.zeros(0, np.int64)
    within = np.arange(cursor, dtype=np.int64) - np.repeat(start[ordered], counts) if ordered else np.zeros(0, np.int64)
    positions = node_pos0 + within

    sub_end = end.copy()
    for n in reversed(order):
        for c in nodes[n].children:
            sub_end[n] = max(sub_end[n], sub_end[c])
    subtree_end = np.repeat(sub_end[ordered], counts) if ordered else np.zeros(0, np.int64)

    key_ranges: list[list[tuple[int, int]]] = [[] for _ in nodes]
    for n in order:
        p = nodes[n].parent
        inherited = [] if p is None else key_ranges[p][:-1] + [(int(start[p]), int(end[p]))]
        key_ranges[n] = [(s, e) for s, e in inherited if e > s] + [(int(start[n]), int(end[n]))]

    src, tgt, pos = [], [], []
    slot_start = np.zeros(nn, np.int64)
    slot_count = np.zeros(nn, np.int64)
    slots = 0
    for n in order:
        node = nodes[n]
        slot_start[n] = slots
        if not node.tokens:
            continue
        scored = np.asarray(node.scored, bool).copy()
        if node.parent is None:
            scored[0] = False
        j = np.flatnonzero(scored)
        if j.size == 0:
            continue
        p = j + start[n]
        s = p - 1
        if node.parent is not None:
            s = np.where(j == 0, end[node.parent] - 1, s)
        src.append(s)
        pos.append(p)
        tgt.append(np.asarray(node.tokens, np.int64)[j])
        slot_count[n] = j.size
        slots += j.size

    l2s, ltraj = [], []
    for traj in forest.trajectories:
        total = 0
        for n in forest.path_to_root(forest.leaf_of[traj.traj_id]):
            c = int(slot_count[n])
            if c:
                l2s.append(np.arange(slot_start[n], slot_start[n] + c, dtype=np.int64))
                total += c
        if total:
            ltraj.append(np.full(total, traj.traj_id, np.int64))

    dev = torch.device(device)

    def t(a) -> torch.Tensor:
        arr = np.concatenate(a) if isinstance(a, list) else a
        if isinstance(a, list) and not a:
            arr = np.zeros(0, np.int64)
        return torch.as_tensor(np.ascontiguousarray(arr, dtype=np.int64)).to(dev)

    parents = np.array([-1 if n.parent is None else n.parent for n in nodes], np.int64)
    depths = np.array([n.depth for n in nodes], np.int64)
    return ExecutionPlan(
        token_ids=t(tokens), position_ids=t(positions), node_of=t(node_of),
        node_start=t(start), node_end=t(end), node_parent=t(parents), node_depth=t(depths),
        subtree_end=t(subtree_end), score_src=t(src), score_tgt=t(tgt), score_pos=t(pos),
        logical_to_slot=t(l2s), logical_traj=t(ltraj), key_ranges=key_ranges, forest=forest,
    )


def visibility_mask(plan: ExecutionPlan) -> torch.Tensor:
    """``[P, P]`` bool mask ``key <= query < subtree_end[key]`` (equal to plan.py:343-362)."""
    p = plan.n_physical
    q = torch.arange(p, device=plan.token_ids.device).unsqueeze(1)
    k = torch.arange(p, device=plan.token_ids.device).unsqueeze(0)
    return (k <= q) & (q < plan.subtree_end.unsqueeze(0))
