"""The dS route's workspace layout (``ts_attn_ds_layout``, CPU).

The dK/dV kernels store dS in blocks of 32 query rows x 16 keys; a (segment,
span) pair keeps, for each 32-row block of the segment, the prefix of the
run's 16-key blocks that some row of it (below q_len) sees, and both kernels
locate a block through a closed-form count of the blocks before its row
block.  The counts are checked here against the definition, enumerated by
brute force over every row block of many rectangles (the diagonal inside,
before and after the run, partial last row blocks and key blocks); the
offsets against their prefix sums in span order, every visit against the
span it names, and the whole layout against the visible pairs it must hold.
"""

from __future__ import annotations

import ctypes
import random

import numpy as np
import pytest
import torch

from thundersync_amd import _abi, _lib
from thundersync_amd import attention as att

pytestmark = pytest.mark.skipif(_lib.library() is None, reason="libthundersync_hip.so not built")

CPU = torch.device("cpu")


def brute_blocks(q_len: int, kv_len: int, kpos: int, run_len: int) -> int:
    """Blocks of one rectangle by definition: row block rb holds key block kb
    when a row r < q_len of it sees key 16 kb of the run (r + kv_len - q_len
    >= kpos + 16 kb)."""
    off = kv_len - q_len
    nkb = (run_len + 15) // 16
    total = 0
    for rb in range((q_len + 31) // 32):
        maxrow = min(32 * rb + 31, q_len - 1)
        total += sum(1 for kb in range(nkb) if kpos + 16 * kb <= off + maxrow)
    return total


def ds_layout(segs, spans, run_len, visits, visit0, nvisit):
    lib = _lib.require_library()
    span_ds = np.zeros(max(len(spans), 1), np.int64)
    visit_ds = np.zeros(max(len(visits), 1), np.int64)
    head = ctypes.c_int64(-1)

    def ptr(a):
        return a.ctypes.data if a.size else None

    st = lib.ts_attn_ds_layout(ptr(segs), len(segs), ptr(spans), len(spans), ptr(run_len), len(run_len),
                               ptr(visits), ptr(visit0), ptr(nvisit), len(visits), span_ds.ctypes.data,
                               visit_ds.ctypes.data, ctypes.byref(head))
    return st, span_ds[: len(spans)], visit_ds[: len(visits)], head.value


def tables(seg_rows, seg_runs, run_len):
    """Host tables for segments (q_len) over run lists; runs in key order."""
    segs = np.zeros(len(seg_rows), _abi.SEG_DTYPE)
    spans, visits_of = [], [[] for _ in run_len]
    row0 = 0
    for s, (q_len, runs) in enumerate(zip(seg_rows, seg_runs)):
        kv = sum(run_len[r] for r in runs)
        segs[s] = (row0, q_len, kv, len(spans), len(runs))
        row0 += q_len
        pos = 0
        for r in runs:
            spans.append((r, pos))
            visits_of[r].append((s, pos))
            pos += run_len[r]
    visits, visit0 = [], []
    for vis in visits_of:
        visit0.append(len(visits))
        visits.extend(vis)
    return (segs, np.array(spans, _abi.REF_DTYPE), np.array(run_len, np.int32), np.array(visits, _abi.REF_DTYPE),
            np.array(visit0, np.int32), np.array([len(v) for v in visits_of], np.int32))


def check(segs, spans, run_len, visits, visit0, nvisit):
    st, span_ds, visit_ds, head = ds_layout(segs, spans, run_len, visits, visit0, nvisit)
    assert st == _lib.TS_OK, _lib.require_library().ts_hip_last_error().decode()
    want, total = [], 0
    for g in segs:
        for i in range(g["nspan"]):
            r, kpos = spans[g["span0"] + i]
            want.append(total)
            total += brute_blocks(int(g["q_len"]), int(g["kv_len"]), int(kpos), int(run_len[r])) * 512
    assert span_ds.tolist() == want
    assert head == total
    for r in range(len(run_len)):
        for v in range(visit0[r], visit0[r] + nvisit[r]):
            s, kpos = visits[v]
            g = segs[s]
            j = [i for i in range(g["nspan"]) if tuple(spans[g["span0"] + i]) == (r, kpos)]
            assert visit_ds[v] == span_ds[g["span0"] + j[0]]
    return head


def test_closed_form_against_the_definition():
    """Many rectangles: q_len 1..200 over runs placed before, across and after
    the diagonal, lengths 1..120 (partial blocks both ways)."""
    rng = random.Random(11)
    run_len = [rng.randint(1, 120) for _ in range(40)]
    seg_rows, seg_runs = [], []
    for _ in range(300):
        runs = rng.sample(range(len(run_len)), rng.randint(1, 4))
        kv = sum(run_len[r] for r in runs)
        seg_rows.append(rng.randint(1, kv))
        seg_runs.append(runs)
    check(*tables(seg_rows, seg_runs, run_len))


@pytest.mark.parametrize("q_len,lens", [(1, [1]), (32, [32]), (33, [17, 16]), (100, [300, 100]), (64, [5, 7, 64]),
                                        (300, [300]), (31, [500, 31])])
def test_edge_shapes(q_len, lens):
    run_len = list(lens)
    check(*tables([q_len], [list(range(len(lens)))], run_len))


def test_layouts_of_the_operators():
    """Chains and retained chunks: each layout's visits name their
    spans' offsets, and the blocks cover every visible pair (at most one
    partial row block and key block of slack per rectangle side)."""
    lays = [att.chain_layout(150, [300, 150], 24, 4), att.chain_layout(200, [300, 17, 200], 40, 8)]
    lays.append(att.retained_chunk_layout(256, [128, 128], [(0, 128, [0]), (128, 128, [0, 1])], 8, 2))
    for lay in lays:
        tabs = lay.device_tables(CPU)
        segs, spans, visits, _, _ = tabs["arrays"]
        run_len = np.array([r.length for r in lay.runs], np.int32)
        head = check(segs, spans, run_len, visits, np.array(tabs["visit0"], np.int32),
                     np.array(tabs["nvisit"], np.int32))
        assert head >= lay.visible_pairs()
        ds = lay.ds_tables(CPU)
        assert ds["head"] == head


def test_refuses_a_visit_that_is_no_span():
    segs, spans, run_len, visits, visit0, nvisit = tables([10], [[0, 1]], [8, 12])
    visits = visits.copy()
    visits[0]["kpos"] = 3
    st, *_ = ds_layout(segs, spans, run_len, visits, visit0, nvisit)
    assert st != _lib.TS_OK and "not a span" in _lib.require_library().ts_hip_last_error().decode()


def test_route_groups_kv_heads_under_the_cap(monkeypatch):
    """The backward's route choice (host side): every KV head per call when
    the whole workspace fits the cap, else as many as fit, else the
    recompute route; head dims without dS kernels and the off switch take
    the recompute route."""
    lib = _lib.require_library()
    lay = att.chain_layout(150, [300, 150], 24, 4)
    head = lay.ds_tables(CPU)["head"]
    q = torch.zeros(150, 24, 256, dtype=torch.bfloat16)
    monkeypatch.setenv(att.DS_ENV, "auto")
    monkeypatch.setattr(att, "DS_FREE_FRACTION", 0.0)  # the cap alone decides
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 1 << 50)
    monkeypatch.setattr(att, "DS_MAX_BYTES", (24 * head + 512) * 2)
    assert att._ds_route(lay, q, lib)[1] == 4
    monkeypatch.setattr(att, "DS_MAX_BYTES", (24 * head + 512) * 2 - 2)
    assert att._ds_route(lay, q, lib)[1] == 3
    monkeypatch.setattr(att, "DS_MAX_BYTES", (6 * head + 512) * 2)
    assert att._ds_route(lay, q, lib)[1] == 1
    monkeypatch.setattr(att, "DS_MAX_BYTES", (6 * head + 512) * 2 - 2)
    assert att._ds_route(lay, q, lib) is None
    monkeypatch.setattr(att, "DS_MAX_BYTES", 16 << 30)
    assert att._ds_route(lay, q[..., :128], lib)[1] == 4
    assert att._ds_route(lay, q[..., :64], lib) is None
    monkeypatch.setenv(att.DS_ENV, "off")
    assert att._ds_route(lay, q, lib) is None


def test_route_takes_free_device_memory_above_the_cap(monkeypatch):
    """A workspace above DS_MAX_BYTES still runs in one call when it fits in
    DS_FREE_FRACTION of the memory the device can supply; with less the route
    falls back to KV-head groups, and with nothing left to the recompute
    route."""
    lib = _lib.require_library()
    lay = att.chain_layout(150, [300, 150], 24, 4)
    head = lay.ds_tables(CPU)["head"]
    need = (24 * head + 512) * 2  # bytes of the one-call workspace
    q = torch.zeros(150, 24, 256, dtype=torch.bfloat16)
    monkeypatch.setenv(att.DS_ENV, "auto")
    monkeypatch.setattr(att, "DS_MAX_BYTES", (6 * head + 512) * 2)  # one KV head
    monkeypatch.setattr(att, "DS_FREE_FRACTION", 0.25)
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 4 * need)
    assert att._ds_route(lay, q, lib)[1] == 4
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 4 * need - 8)
    assert att._ds_route(lay, q, lib)[1] == 3
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 0)
    assert att._ds_route(lay, q, lib) is None


def test_route_never_takes_more_than_half_the_available_memory(monkeypatch):
    """Within DS_MAX_BYTES the workspace is still bounded by
    DS_AVAILABLE_FRACTION of what the device can supply: a nearly full device
    runs fewer KV heads per call, or the recompute route."""
    lib = _lib.require_library()
    lay = att.chain_layout(150, [300, 150], 24, 4)
    head = lay.ds_tables(CPU)["head"]
    need = (24 * head + 512) * 2
    q = torch.zeros(150, 24, 256, dtype=torch.bfloat16)
    monkeypatch.setenv(att.DS_ENV, "auto")
    monkeypatch.setattr(att, "DS_MAX_BYTES", 16 << 30)
    assert need < att.DS_MAX_BYTES and att.DS_AVAILABLE_FRACTION == 0.5
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 2 * need)
    assert att._ds_route(lay, q, lib)[1] == 4
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 2 * need - 8)
    assert att._ds_route(lay, q, lib)[1] == 3
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 2 * (6 * head + 512) * 2)
    assert att._ds_route(lay, q, lib)[1] == 1
    monkeypatch.setattr(att, "_device_free_bytes", lambda device: 2 * (6 * head + 512) * 2 - 8)
    assert att._ds_route(lay, q, lib) is None
