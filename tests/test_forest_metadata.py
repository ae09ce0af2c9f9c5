"""Packing / segment-index metadata, bit-exact (CPU).

Three-way check: the reference's own outputs (golden vectors written by
tests/golden/make_forest_golden.py from engine/segments.py and
engine/plan.py), the oracle's step-for-step restatement, and the product
builder in thundersync_amd.forest.  Larger random forests compare product
against oracle and check the invariants the reference's tests assert
(a trajectory's physical path reproduces it; the subtree-end rule equals
the dense visibility mask).
"""

from __future__ import annotations

import json
import random
from pathlib import Path

import pytest
import torch

from oracle import forest as ref
from thundersync_amd import forest as prod
from thundersync_amd.attention import pack_layout

GOLDEN = json.loads((Path(__file__).parent / "golden" / "forest_metadata.json").read_text())
FIELDS = ("token_ids", "position_ids", "node_of", "node_start", "node_end", "node_parent", "node_depth",
          "subtree_end", "score_src", "score_tgt", "score_pos", "logical_to_slot", "logical_traj")


def _oracle_trajs(spec):
    return [ref.Trajectory([ref.Segment(tuple(toks), kind, scored) for kind, toks, scored in segs], g, t)
            for g, t, segs in spec]


def _prod_trajs(spec):
    kinds = {"prompt": prod.SegmentKind.PROMPT, "action": prod.SegmentKind.ACTION,
             "observation": prod.SegmentKind.OBSERVATION}
    return [prod.Trajectory([prod.Segment(tuple(toks), kinds[kind], scored) for kind, toks, scored in segs],
                            group_id=g, traj_id=t) for g, t, segs in spec]


def _forest_dict(forest):
    return {
        "nodes": [{"tokens": n.tokens, "scored": n.scored, "parent": n.parent, "depth": n.depth,
                   "trajectories": n.trajectories, "children": n.children, "group_id": n.group_id}
                  for n in forest.nodes],
        "roots": forest.roots,
        "leaf_of": {str(k): v for k, v in forest.leaf_of.items()},
    }


def _plan_dict(plan):
    if isinstance(plan, dict):
        return plan
    out = {f: getattr(plan, f).tolist() for f in FIELDS}
    out["key_ranges"] = [[list(r) for r in kr] for kr in plan.key_ranges]
    return out


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_oracle_matches_reference_golden(name):
    case = GOLDEN[name]
    forest = ref.build_forest(_oracle_trajs(case["trajectories"]))
    assert _forest_dict(forest) == case["forest"]
    plan = ref.compile_plan(forest)
    assert _plan_dict(plan) == case["plan"]
    mask = ref.visibility_mask(plan)
    assert ["".join("1" if b else "0" for b in row) for row in mask] == case["visibility_mask_rows"]


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_product_matches_reference_golden(name):
    case = GOLDEN[name]
    forest = prod.build_forest(_prod_trajs(case["trajectories"]))
    assert _forest_dict(forest) == case["forest"]
    plan = prod.compile_plan(forest)
    assert _plan_dict(plan) == case["plan"]
    for f in FIELDS:
        assert getattr(plan, f).dtype == torch.int64
    mask = prod.visibility_mask(plan)
    assert ["".join("1" if b else "0" for b in row) for row in mask.tolist()] == case["visibility_mask_rows"]


def _random_spec(seed, groups=3, per_group=5, prompt=(1, 30), turns=4, vocab=5):
    rng = random.Random(seed)
    spec, tid = [], 0
    for g in rng.sample(range(10), groups):
        p = [rng.randrange(vocab) for _ in range(rng.randint(*prompt))]
        for _ in range(per_group):
            segs = [["prompt", p, False]]
            for _ in range(rng.randint(1, turns)):
                segs.append(["action", [rng.randrange(vocab) for _ in range(rng.randint(1, 4))], True])
                if rng.random() < 0.7:
                    segs.append(["observation", [rng.randrange(vocab) for _ in range(rng.randint(1, 3))], False])
            spec.append([g, tid, segs])
            tid += 1
    rng.shuffle(spec)
    return spec


@pytest.mark.parametrize("seed", range(12))
def test_product_matches_oracle_on_random_forests(seed):
    spec = _random_spec(seed)
    o_forest = ref.build_forest(_oracle_trajs(spec))
    p_forest = prod.build_forest(_prod_trajs(spec))
    assert _forest_dict(p_forest) == _forest_dict(o_forest)
    o_plan = ref.compile_plan(o_forest)
    p_plan = prod.compile_plan(p_forest)
    assert _plan_dict(p_plan) == _plan_dict(o_plan)
    # invariants the reference's tests assert
    for g, tid, segs in spec:
        path = p_plan.physical_path(tid)
        toks = [t for _k, ts, _s in segs for t in ts]
        assert p_plan.token_ids[path].tolist() == toks
        assert p_plan.position_ids[path].tolist() == list(range(len(toks)))
    dense = ref.visibility_mask(o_plan)
    assert prod.visibility_mask(p_plan).tolist() == dense


def test_forest_shapes_of_the_benchmark_configs():
    """C2: one prompt shared by 8 completions; C4: 4 groups x 4, distinct tokens."""
    rng = random.Random(0)
    prompt = [rng.randrange(1000) for _ in range(2048)]
    trajs = [prod.Trajectory([prod.Segment.prompt(prompt),
                              prod.Segment.action([1000 + i] + [rng.randrange(1000) for _ in range(300)])],
                             group_id=0, traj_id=i) for i in range(8)]
    plan = prod.compile_plan(prod.build_forest(trajs))
    assert plan.n_nodes == 9 and plan.is_two_level
    assert plan.node_start.tolist()[0] == 0 and plan.node_end.tolist()[0] == 2048
    assert all(kr[0] == (0, 2048) for kr in plan.key_ranges[1:])


PACK_GOLDEN = json.loads((Path(__file__).parent / "golden" / "pack_layout.json").read_text())


def test_pack_layout_cumulative_lengths():
    lengths = [157, 157, 42, 157]
    ancestors = [
        ([torch.zeros(n, 1, 1) for n in chunks], [torch.zeros(n, 1, 1) for n in chunks])
        for chunks in ([492, 157, 157], [492, 42, 157, 68], [492], [492, 157])
    ]
    layout = pack_layout(lengths, ancestors)
    prefixes = [sum(c.shape[0] for c in ks) for ks, _ in ancestors]
    cu_l, cu_p = ref.pack_cumulative(lengths, prefixes)
    assert layout.cu_lengths.dtype == torch.int32 and layout.cu_lengths.tolist() == cu_l
    assert layout.cu_prefixes.dtype == torch.int32 and layout.cu_prefixes.tolist() == cu_p
    assert layout.prefixes == prefixes and layout.counts == [3, 4, 1, 2]
    assert cu_l == [0, 157, 314, 356, 513] and cu_p == [0, 806, 1565, 2057, 2706]


def _tagged_ancestors(counts):
    """One distinct tensor per (half, segment, chunk); identity says which."""
    return [([torch.zeros(c + 1, 1, 1) for c in range(n)], [torch.zeros(c + 1, 1, 1) for c in range(n)])
            for n in counts]


@pytest.mark.parametrize("name", sorted(PACK_GOLDEN))
def test_pack_layout_input_order_matches_reference(name):
    """PackLayout.inputs / by_segment against the order the reference's own
    _PackLayout produced (engine/streaming.py:1636-1650; fixture written by
    tests/golden/make_pack_golden.py)."""
    case = PACK_GOLDEN[name]
    counts = case["counts"]
    ancestors = _tagged_ancestors(counts)
    layout = pack_layout([1] * len(counts), ancestors)
    assert layout.counts == counts
    inputs = layout.inputs(ancestors)
    assert len(inputs) == len(case["inputs"])
    for got, (half, s, c) in zip(inputs, case["inputs"]):
        assert got is ancestors[s][half][c]
    total = sum(counts)
    regrouped = layout.by_segment(tuple(inputs[:total]))
    assert [len(seg) for seg in regrouped] == [len(seg) for seg in case["by_segment"]]
    for seg, positions in zip(regrouped, case["by_segment"]):
        assert all(a is inputs[p] for a, p in zip(seg, positions))


@pytest.mark.parametrize("name", sorted(PACK_GOLDEN))
def test_oracle_pack_input_order_matches_reference(name):
    case = PACK_GOLDEN[name]
    order = ref.pack_input_order(case["counts"])
    total = sum(case["counts"])
    assert [[0, s, c] for s, c in order] == case["inputs"][:total]
    assert [[1, s, c] for s, c in order] == case["inputs"][total:]


@pytest.mark.parametrize("name", sorted(GOLDEN))
def test_plan_from_node_lists_matches_golden(name):
    """compile_plan on a forest that does not carry the builder's flat keys
    (a forest assembled from node lists, as the reference's builder returns)."""
    case = GOLDEN[name]
    forest = prod.build_forest(_prod_trajs(case["trajectories"]))
    forest._flat = None
    assert _plan_dict(prod.compile_plan(forest)) == case["plan"]


def test_empty_batch():
    forest = prod.build_forest([])
    assert forest.nodes == [] and forest.roots == [] and forest.leaf_of == {}
    plan = prod.compile_plan(forest)
    assert plan.n_physical == 0 and plan.n_scored == 0 and plan.n_nodes == 0
    assert plan.logical_to_slot.numel() == 0 and plan.key_ranges == []


def test_native_builder_rejects_bad_arguments():
    """The C entry points report bad input as an error status (host code only)."""
    import ctypes

    import numpy as np

    from thundersync_amd import _lib

    lib = _lib.require_library()
    p = lambda a: a.ctypes.data
    keys = np.array([4, 6, 4, 8], np.int64)
    offsets = np.array([0, 2, 4], np.int64)
    groups = np.zeros(2, np.int64)
    out = [np.zeros(4, np.int64) for _ in range(6)]
    leaf = np.zeros(2, np.int64)
    count = ctypes.c_int64(0)
    args = (p(groups), p(offsets), p(keys))
    assert lib.ts_forest_build(2, *args, 3, ctypes.byref(count), *map(p, out), p(leaf)) == 1
    assert b"max_nodes" in lib.ts_hip_last_error()
    assert lib.ts_forest_build(2, *args, 4, ctypes.byref(count), *map(p, out), p(leaf)) == 0
    assert count.value == 3 and out[0][:3].tolist() == [-1, 0, 0] and leaf.tolist() == [1, 2]
    empty = np.array([0, 2, 2], np.int64)
    assert lib.ts_forest_build(2, p(groups), p(empty), p(keys), 4, ctypes.byref(count), *map(p, out), p(leaf)) == 1
    assert b"empty" in lib.ts_hip_last_error()
    # a plan whose order lists a child before its parent
    parent = np.array([-1, 0], np.int64)
    bad_order = np.array([1, 0], np.int64)
    lens = np.array([1, 1], np.int64)
    koff = np.array([0, 1], np.int64)
    bufs = [np.zeros(4, np.int64) for _ in range(11)]
    n1, n2 = ctypes.c_int64(0), ctypes.c_int64(0)
    one = np.array([1], np.int64)
    status = lib.ts_plan_compile(2, p(parent), p(bad_order), p(lens), p(koff), p(keys), 1, p(one), p(one), 4,
                                 *map(p, bufs[:9]), ctypes.byref(n1), p(bufs[9]), p(bufs[10]), ctypes.byref(n2))
    assert status == 1 and b"before its parent" in lib.ts_hip_last_error()
