"""The attention layouts' integer work lists (CPU).

Every dK/dV work item is one ``kv_block`` of keys of one visited run, and its
cost is the number of query rows of its visits that see the block's first
key; every forward/dQ item is one ``q_block`` of rows of one segment, and its
cost is the number of keys its last row sees.  Both lists run in geometric
cost bands of width ORDER_BAND, longest band first, and within a band in
(segment or run, first row or key) order.  Here they are recomputed item by
item and compared with the layout's tables, on the bench layouts and on
random retained-chunk packs.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from thundersync_amd import attention as att


def expected_lists(lay):
    qb = att.q_block_rows(lay.hq, lay.hkv)
    kvb = att.kv_block_keys(lay.hq, lay.hkv)
    q_items = []
    for s, (row0, n) in enumerate(lay.seg_q):
        off = lay.seg_kv[s] - n
        for q0 in range(0, n, qb):
            q_items.append((-(off + min(q0 + qb, n)), s, q0))
    visits = [[] for _ in lay.runs]
    for s, spans in enumerate(lay.seg_spans):
        for run, kpos in spans:
            visits[run].append((s, kpos))
    kv_items = []
    for run, vis in enumerate(visits):
        if not vis:
            continue
        for k0 in range(0, lay.runs[run].length, kvb):
            cost = 0
            for s, kpos in vis:
                n = lay.seg_q[s][1]
                first = max(0, kpos + k0 - (lay.seg_kv[s] - n))
                cost += max(0, n - first)
            kv_items.append((-cost, run, k0))
    def band(cost):
        return int(np.floor(np.log(np.float64(max(cost, 1))) / np.log(1.0 + att.ORDER_BAND)))

    q_items.sort(key=lambda x: (-band(-x[0]), x[1], x[2]))
    kv_items.sort(key=lambda x: (-band(-x[0]), x[1], x[2]))
    return [(s, q0) for _, s, q0 in q_items], [(r, k0) for _, r, k0 in kv_items]


def check(lay):
    _, _, _, q_work, kv_work, *_ = lay._host_tables()
    want_q, want_kv = expected_lists(lay)
    assert q_work.dtype == np.int32 and kv_work.dtype == np.int32
    assert [tuple(x) for x in q_work.tolist()] == want_q
    assert [tuple(x) for x in kv_work.tolist()] == want_kv


def test_bench_layouts():
    import bench

    plan, *_ = bench.c2_inputs(0, torch.device("cpu"))
    check(att.forest_layout(plan, 32, 8))
    _, chunk_rows, chunks, rows = bench.c4_layout(0)
    check(att.retained_chunk_layout(rows, chunk_rows, chunks, 32, 8))


@pytest.mark.parametrize("hq,hkv", [(32, 8), (40, 8), (8, 2), (4, 4)])
@pytest.mark.parametrize("seed", range(4))
def test_random_packs(seed, hq, hkv):
    import bench

    rng = random.Random(seed)
    _, chunk_rows, chunks, rows = bench.c4_layout(seed, chunk=rng.choice([64, 100, 512]), groups=2, per_group=3,
                                                  prompt=rng.randint(1, 700), lo=1, hi=900)
    check(att.retained_chunk_layout(rows, chunk_rows, chunks, hq, hkv))


def test_head_dim_256_item_size_follows_the_item_count():
    """At head dim 256 the dK/dV items hold 64 keys (two waves of 32 keys)
    unless their count over all KV heads is below DKDV256_MIN_ITEMS, then 48
    (the key-split kernel); other head dims keep ts_attn_kv_block's size, and
    each size has its own work list."""
    cpu = torch.device("cpu")
    big = att.chain_layout(9288, [3000, 9288], 24, 4)  # (47 + 146) x 4 = 772 items of 64 keys
    small = att.chain_layout(100, [300, 100], 24, 4)  # (5 + 2) x 4 = 28
    group4 = att.chain_layout(9288, [3000, 9288], 16, 4)
    assert big.kv_block_for(cpu, 256) == 64 and small.kv_block_for(cpu, 256) == 48
    assert big.kv_block_for(cpu, 128) == 64 and group4.kv_block_for(cpu, 128) == 48
    assert group4.kv_block_for(cpu, 256) == 64
    for kvb in (48, 64):
        kv_work = big.device_tables(cpu, kvb)["arrays"][4]
        assert len(kv_work) == sum(-(-n // kvb) for n in (3000, 9288))
        assert set(kv_work[:, 1].tolist()) <= set(range(0, 9288, kvb))
