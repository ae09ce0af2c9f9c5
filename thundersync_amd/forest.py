"""Segment forest and execution plan: the integer metadata the kernels consume.

Same API and bit-identical outputs as the reference's
``engine/segments.py`` (``Segment``, ``Trajectory``, ``build_forest``) and
``engine/plan.py`` (``ExecutionPlan``, ``compile_plan``,
``visibility_mask``), built differently: the trie and the plan arrays are
computed in native code (``ts_forest_build``, ``ts_plan_compile``) in one pass
over flat ``2 * token + scored`` key arrays -- an explicit work stack and
direct mismatch scans instead of recursion and binary search over slices --
and this module only packs the keys and wraps the results in the reference's
objects.  The conventions that make the output bit-exact are kept:

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

import ctypes

import numpy as np
import torch

from . import _lib


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

    @property
    def padded_tokens(self) -> int:
        """Tokens of the [trajectories, longest] rectangle a padded batch would hold."""
        return len(self.trajectories) * max((t.n_tokens for t in self.trajectories), default=0)

    def path_to_root(self, node: int) -> list[int]:
        path = []
        cur: int | None = node
        while cur is not None:
            path.append(cur)
            cur = self.nodes[cur].parent
        return path[::-1]


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _flat_keys(trajectories: Sequence[Trajectory]) -> tuple[np.ndarray, np.ndarray]:
    parts = [t.keys() for t in trajectories]
    offsets = np.zeros(len(parts) + 1, np.int64)
    np.cumsum([len(p) for p in parts], out=offsets[1:])
    keys = np.ascontiguousarray(np.concatenate(parts), np.int64) if parts else np.zeros(1, np.int64)
    return keys, offsets


def build_forest(trajectories: Sequence[Trajectory]) -> SegmentForest:
    """Compress trajectories into the exact shared forest (segments.py:280-346 semantics),
    on ``ts_forest_build``."""
    trajs = list(trajectories)
    lib = _lib.require_library()
    n = len(trajs)
    keys, offsets = _flat_keys(trajs)
    groups = np.array([t.group_id for t in trajs] or [0], np.int64)
    cap = max(2 * n, 1)
    parent, depth, group, src, off, length = (np.zeros(cap, np.int64) for _ in range(6))
    leaf = np.zeros(max(n, 1), np.int64)
    count = ctypes.c_int64(0)
    _lib.check(lib.ts_forest_build(n, _ptr(groups), _ptr(offsets), _ptr(keys), cap, ctypes.byref(count),
                                   _ptr(parent), _ptr(depth), _ptr(group), _ptr(src), _ptr(off), _ptr(length),
                                   _ptr(leaf)), f"ts_forest_build({n} trajectories)")
    nn = count.value
    parents = parent[:nn].tolist()
    starts = (offsets[src[:nn]] + off[:nn]).tolist()
    lens = length[:nn].tolist()
    members: list[list[int]] = [[] for _ in range(nn)]
    leaf_of: dict[int, int] = {}
    for i, t in enumerate(trajs):
        node = int(leaf[i])
        leaf_of[t.traj_id] = node
        while node >= 0:
            members[node].append(t.traj_id)
            node = parents[node]
    nodes: list[ForestNode] = []
    roots: list[int] = []
    for idx in range(nn):
        head = keys[starts[idx]:starts[idx] + lens[idx]]
        p = parents[idx]
        nodes.append(ForestNode(tokens=(head >> 1).tolist(), scored=(head & 1).astype(bool).tolist(),
                                parent=None if p < 0 else p, depth=int(depth[idx]), trajectories=members[idx],
                                group_id=int(group[idx])))
        if p < 0:
            roots.append(idx)
        else:
            nodes[p].children.append(idx)
    forest = SegmentForest(nodes, roots, trajs, leaf_of)
    forest._flat = (keys, np.asarray(starts, np.int64), np.asarray(lens, np.int64))
    return forest


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


def _node_keys(forest: SegmentForest) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(keys, node key offsets, node lengths): the builder's flat keys when the
    nodes still match them, else the nodes' own token lists packed as keys."""
    lengths = np.array([len(n.tokens) for n in forest.nodes], np.int64)
    flat = getattr(forest, "_flat", None)
    if flat is not None and flat[2].shape == lengths.shape and np.array_equal(flat[2], lengths):
        return flat[0], flat[1], lengths
    parts = [np.asarray(n.tokens, np.int64) * 2 + np.asarray(n.scored, np.int64) for n in forest.nodes]
    offsets = np.zeros(len(parts), np.int64)
    if parts:
        np.cumsum(lengths[:-1], out=offsets[1:])
    keys = np.concatenate(parts) if parts and lengths.sum() else np.zeros(1, np.int64)
    return np.ascontiguousarray(keys, np.int64), offsets, lengths


def compile_plan(forest: SegmentForest, device: torch.device | str = "cpu") -> ExecutionPlan:
    """Lay the forest out in DFS pre-order and derive every index from it
    (plan.py:166-340), on ``ts_plan_compile``."""
    lib = _lib.require_library()
    nodes = forest.nodes
    nn = len(nodes)
    order_list = _preorder(forest)
    order = np.asarray(order_list or [0], np.int64)
    keys, key_off, lengths = _node_keys(forest)
    parents = np.array([-1 if n.parent is None else n.parent for n in nodes] or [0], np.int64)
    p_total = int(lengths.sum())
    trajs = forest.trajectories
    traj_leaf = np.array([forest.leaf_of[t.traj_id] for t in trajs] or [0], np.int64)
    traj_ids = np.array([t.traj_id for t in trajs] or [0], np.int64)
    max_logical = sum(t.n_tokens for t in trajs)
    cap_p, cap_l = max(p_total, 1), max(max_logical, 1)
    token_ids, position_ids, node_of, subtree_end, src, tgt, pos = (np.zeros(cap_p, np.int64) for _ in range(7))
    start, end = np.zeros(max(nn, 1), np.int64), np.zeros(max(nn, 1), np.int64)
    l2s, ltraj = np.zeros(cap_l, np.int64), np.zeros(cap_l, np.int64)
    n_scored, n_logical = ctypes.c_int64(0), ctypes.c_int64(0)
    _lib.check(lib.ts_plan_compile(nn, _ptr(parents), _ptr(order), _ptr(np.ascontiguousarray(lengths if nn else order)),
                                   _ptr(np.ascontiguousarray(key_off if nn else order)), _ptr(keys), len(trajs),
                                   _ptr(traj_leaf), _ptr(traj_ids), max_logical, _ptr(token_ids), _ptr(position_ids),
                                   _ptr(node_of), _ptr(start), _ptr(end), _ptr(subtree_end), _ptr(src), _ptr(tgt),
                                   _ptr(pos), ctypes.byref(n_scored), _ptr(l2s), _ptr(ltraj), ctypes.byref(n_logical)),
               f"ts_plan_compile({nn} nodes, {p_total} rows)")
    ns, nl = n_scored.value, n_logical.value

    starts, ends = start[:nn].tolist(), end[:nn].tolist()
    key_ranges: list[list[tuple[int, int]]] = [[] for _ in nodes]
    for n in order_list:
        p = nodes[n].parent
        inherited = [] if p is None else key_ranges[p][:-1] + [(starts[p], ends[p])]
        key_ranges[n] = [(s, e) for s, e in inherited if e > s] + [(starts[n], ends[n])]

    dev = torch.device(device)

    def t(a: np.ndarray, count: int) -> torch.Tensor:
        return torch.from_numpy(a[:count].copy()).to(dev)

    depths = np.array([n.depth for n in nodes], np.int64)
    return ExecutionPlan(
        token_ids=t(token_ids, p_total), position_ids=t(position_ids, p_total), node_of=t(node_of, p_total),
        node_start=t(start, nn), node_end=t(end, nn), node_parent=t(parents, nn), node_depth=t(depths, nn),
        subtree_end=t(subtree_end, p_total), score_src=t(src, ns), score_tgt=t(tgt, ns), score_pos=t(pos, ns),
        logical_to_slot=t(l2s, nl), logical_traj=t(ltraj, nl), key_ranges=key_ranges, forest=forest,
    )


def visibility_mask(plan: ExecutionPlan) -> torch.Tensor:
    """``[P, P]`` bool mask ``key <= query < subtree_end[key]`` (equal to plan.py:343-362)."""
    p = plan.n_physical
    q = torch.arange(p, device=plan.token_ids.device).unsqueeze(1)
    k = torch.arange(p, device=plan.token_ids.device).unsqueeze(0)
    return (k <= q) & (q < plan.subtree_end.unsqueeze(0))
