"""The host-side table check of the attention entry points (CPU).

``ts_attn_check_tables`` reads host copies of a problem's tables.  The
layouts the operators build (bench forest and retained-chunk layouts, random
packs, ragged cohorts, chunk chains) pass it; each inconsistency planted
below (a repeated or missing work item, a span off its position, a visit that
no segment spans, an unaligned or empty run, rows outside the query tensor)
is refused with a message that names it.  Nothing launches: the run table
holds made-up aligned addresses.
"""

from __future__ import annotations

import ctypes
import random

import numpy as np
import pytest
import torch

from thundersync_amd import _lib
from thundersync_amd import attention as att

pytestmark = pytest.mark.skipif(_lib.library() is None, reason="libthundersync_hip.so not built")

CPU = torch.device("cpu")


def fake_runs(lay, *, grads=True):
    """A run table with distinct 16-byte aligned addresses and packed strides."""
    table = np.zeros(len(lay.runs), att.RUN_DTYPE)
    row = lay.hkv * att.HEAD_DIM
    for r, run in enumerate(lay.runs):
        base = (1 << 40) + (run.source << 32) + run.offset * row * 2
        t = table[r]
        t["k"], t["v"] = base, base + (1 << 30)
        t["k_row_stride"] = t["v_row_stride"] = row
        t["k_head_stride"] = t["v_head_stride"] = att.HEAD_DIM
        if grads:
            t["dk"], t["dv"] = base + (2 << 30), base + (3 << 30)
            t["dk_row_stride"] = t["dv_row_stride"] = row
            t["dk_head_stride"] = t["dv_head_stride"] = att.HEAD_DIM
        t["len"] = run.length
    tabs = lay.device_tables(CPU)
    table["visit0"] = tabs["visit0"]
    table["nvisit"] = tabs["nvisit"]
    return table


def run_check(lay, *, runs=None, arrays=None, **problem_fields):
    """Status and message of the check on (possibly altered) host tables."""
    segs, spans, visits, q_work, kv_work = arrays or lay.device_tables(CPU)["arrays"]
    runs = fake_runs(lay) if runs is None else runs
    problem = lay.problem(CPU, 1 << 20, 0.125)
    for name, value in problem_fields.items():
        setattr(problem, name, value)
    lib = _lib.require_library()

    def ptr(a):
        return a.ctypes.data if a.size else None

    status = lib.ts_attn_check_tables(ctypes.byref(problem), ptr(segs), ptr(spans), spans.shape[0], ptr(runs),
                                      ptr(visits), visits.shape[0], ptr(q_work), ptr(kv_work))
    return status, lib.ts_hip_last_error().decode() if status else ""


def layouts():
    import bench

    plan, *_ = bench.c2_inputs(0, CPU)
    yield "c2_forest", att.forest_layout(plan, 32, 8)
    _, chunk_rows, chunks, rows = bench.c4_layout(0)
    yield "c4_chunks", att.retained_chunk_layout(rows, chunk_rows, chunks, 32, 8)
    for seed in range(3):
        rng = random.Random(seed)
        hq, hkv = rng.choice([(32, 8), (40, 8), (8, 2), (4, 4)])
        _, chunk_rows, chunks, rows = bench.c4_layout(seed, chunk=rng.choice([64, 100, 512]), groups=2,
                                                      per_group=3, prompt=rng.randint(1, 700), lo=1, hi=900)
        yield f"pack{seed}", att.retained_chunk_layout(rows, chunk_rows, chunks, hq, hkv)
    yield "ragged", att._ragged_layout([5, 0, 130, 64], [9, 3, 130, 200], 8, 2)
    yield "chain", att.chain_layout(300, [128, 77, 300], 16, 4)


@pytest.mark.parametrize("name,lay", list(layouts()), ids=lambda x: x if isinstance(x, str) else "")
def test_operator_layouts_pass(name, lay):
    assert run_check(lay) == (0, "")
    # the forward's run table (no gradient destinations) passes as well
    assert run_check(lay, runs=fake_runs(lay, grads=False)) == (0, "")


def test_python_wrapper_checks_and_raises():
    lay = att.chain_layout(64, [64, 64], 8, 2)
    problem = lay.problem(CPU, 1 << 20, 0.1)
    att.check_tables(lay, problem, fake_runs(lay), CPU)
    bad = fake_runs(lay)
    bad[1]["k"] += 8
    with pytest.raises(RuntimeError, match="run 1 K/V need 16-byte aligned rows"):
        att.check_tables(lay, problem, bad, CPU)
    with pytest.raises(ValueError, match="run table"):
        att.check_tables(lay, problem, bad[:1], CPU)


def copies(lay):
    return [a.copy() for a in lay.device_tables(CPU)["arrays"]]


@pytest.fixture
def pack():
    import bench

    _, chunk_rows, chunks, rows = bench.c4_layout(1, chunk=100, groups=2, per_group=3, prompt=300, lo=1, hi=500)
    return att.retained_chunk_layout(rows, chunk_rows, chunks, 32, 8)


def test_repeated_forward_item(pack):
    segs, spans, visits, q_work, kv_work = copies(pack)
    q_work[1] = q_work[0]
    status, msg = run_check(pack, arrays=(segs, spans, visits, q_work, kv_work))
    assert status != 0 and "repeats segment" in msg


def test_missing_key_block(pack):
    status, msg = run_check(pack, n_kv_work=pack.device_tables(CPU)["n_kv_work"] - 1, n_kv_long=0)
    assert status != 0 and "dK/dV items for" in msg


def test_misaligned_forward_item(pack):
    segs, spans, visits, q_work, kv_work = copies(pack)
    q_work[0, 1] += 1
    status, msg = run_check(pack, arrays=(segs, spans, visits, q_work, kv_work))
    assert status != 0 and "is not a row block" in msg


def test_key_item_of_an_unvisited_run():
    lay = att.AttnLayout(q_rows=8, hq=8, hkv=2, source_rows=(64, 64), runs=(att.Run(0, 0, 64), att.Run(1, 0, 64)),
                         seg_q=((0, 8),), seg_spans=(((0, 0),),))
    segs, spans, visits, q_work, kv_work = copies(lay)
    kv_work[0] = (1, 0)
    status, msg = run_check(lay, arrays=(segs, spans, visits, q_work, kv_work))
    assert status != 0 and "not a key block of a visited run" in msg


def test_span_off_its_position(pack):
    segs, spans, visits, q_work, kv_work = copies(pack)
    s = next(i for i in range(len(segs)) if segs[i]["nspan"] > 1)
    spans[segs[s]["span0"] + 1]["kpos"] += 1
    status, msg = run_check(pack, arrays=(segs, spans, visits, q_work, kv_work))
    assert status != 0 and f"segment {s} span 1 at key" in msg


def test_visit_without_a_span(pack):
    segs, spans, visits, q_work, kv_work = copies(pack)
    visits[0]["kpos"] += 1
    status, msg = run_check(pack, arrays=(segs, spans, visits, q_work, kv_work))
    assert status != 0 and "is not a span of that segment" in msg


def test_repeated_visit(pack):
    segs, spans, visits, q_work, kv_work = copies(pack)
    runs = fake_runs(pack)
    r = int(np.flatnonzero(runs["nvisit"] > 1)[0])
    v0 = runs[r]["visit0"]
    visits[v0 + 1] = visits[v0]
    status, msg = run_check(pack, runs=runs, arrays=(segs, spans, visits, q_work, kv_work))
    assert status != 0 and f"run {r} visit 1 repeats segment" in msg


def test_visit_count_mismatch(pack):
    runs = fake_runs(pack)
    r = int(np.flatnonzero(runs["nvisit"] > 1)[0])
    runs[r]["nvisit"] -= 1
    status, msg = run_check(pack, runs=runs)
    assert status != 0 and ("visits for" in msg or "dK/dV items" in msg)


def test_segment_rows_outside_the_query(pack):
    segs, spans, visits, q_work, kv_work = copies(pack)
    segs[-1]["q_row0"] = pack.q_rows - segs[-1]["q_len"] + 1
    status, msg = run_check(pack, arrays=(segs, spans, visits, q_work, kv_work))
    assert status != 0 and "outside [0," in msg


def test_empty_run_and_bad_strides(pack):
    runs = fake_runs(pack)
    runs[0]["len"] = 0
    status, msg = run_check(pack, runs=runs)
    assert status != 0 and "run 0 has length 0" in msg
    runs = fake_runs(pack)
    runs[2]["v_row_stride"] = 1 << 24
    status, msg = run_check(pack, runs=runs)
    assert status != 0 and "run 2 K/V" in msg
    runs = fake_runs(pack)
    runs[3]["dv"] += 2
    status, msg = run_check(pack, runs=runs)
    assert status != 0 and "run 3 dK/dV" in msg


def test_problem_fields(pack):
    status, msg = run_check(pack, q_block=64)
    assert status != 0 and "q_block" in msg
    status, msg = run_check(pack, n_q_long=pack.device_tables(CPU)["n_q_work"] + 1)
    assert status != 0 and "long-item counts" in msg
