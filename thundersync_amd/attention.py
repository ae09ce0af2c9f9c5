"""Forest / packed bottom-right-causal GQA attention on the gfx950 kernels.

One differentiable core op, :func:`attention`, serves every shape the
reference's streaming engine produces.  A call is described by an
:class:`AttnLayout`:

* **key sources** -- the K/V tensors the call reads, each ``[N, Hkv, D]``
  (a retained chunk, a pack's own K/V, a forest's whole K/V), read in place;
* **runs** -- contiguous row ranges of a source (a whole chunk, one forest
  node);
* **segments** -- blocks of query rows of the packed ``[R, Hq, D]`` query,
  each attending bottom-right-causally to the concatenation of its runs.

The layout is integer metadata only (no pointers), so one layout serves every
layer of a model call, as the reference's ``_PackLayout`` does
(src/thundersync/engine/streaming.py:1613-1698).  The pointer table is
rebuilt per call from the tensors themselves.

Reference entry points mirrored here (same argument meaning):

* :func:`causal_attention` -- the callable-backend form ``(query, ks, vs,
  scale) -> out`` that ``_causal_sdpa(..., backend=)`` dispatches to
  (engine/streaming.py:1094-1095) and ``grpo/attention.py:148-172`` provides;
* :class:`ChunkedCausalAttention` -- ``_ChunkedCausalSDPA.apply(query, scale,
  n_chunks, keep_state, backend, *ks, *vs)`` (engine/streaming.py:1314-1423);
* :class:`PackLayout` / :class:`PackedAttention` -- ``_PackedFlashSplit.apply(
  query, key, value, scale, layout, *ancestors)`` (engine/streaming.py:
  1613-1836), with ancestors in the reference's "last segment first" order;
* :func:`ragged_causal_attention` -- ``_ragged_causal_sdpa`` (:1165-1226),
  and :class:`RaggedAttention` -- ``_RaggedAttentionIndependentVJP``
  (:1253-1297);
* :func:`forest_attention` -- ``forest_attention(q, k, v, plan, *, scale)``
  (engine/attention.py:186-231);
* :func:`retained_chunk_layout` / :func:`retained_chunk_attention` -- every
  query chunk of a streamed pack over its retained per-chunk K/V in one
  launch, each chunk being the call ``_ChunkedCausalSDPA`` makes
  (engine/streaming.py:1314-1423).

Element types: bf16 and fp16 (Q, K, V of one call share one).  Head dims D:
any from 1 to 256, as the reference's flash paths take
(engine/streaming.py:532-548, :915-930).  The kernels are built for 32, 64,
96, 128, 192 and 256 (128 and 256 run the DMA-staged kernels, the others the
register-staged ones); any other D runs the next larger of them over Q, K
and V zero-padded to it (see :func:`kernel_head_dim`).  At head dims 128 and
256 the backward stores dS once in a workspace and forms dQ = dS K from it
(see ``DS_MAX_BYTES``).  There is no host path: CPU tensors, other dtypes or
head dims above 256 raise.
"""

from __future__ import annotations

import ctypes
import math
import os
import threading
from collections.abc import Sequence
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from ._abi import REF_DTYPE, RUN_DTYPE, SEG_DTYPE, AttnProblem, AttnRows
from .dispatch import HIP_BACKWARD_PATH, HIP_PATH, count_attention_path
from .operator_profiling import operator_range

HEAD_DIMS = (32, 64, 96, 128, 192, 256)  # the head dims the kernels are built for
MAX_HEAD_DIM = 256
HEAD_DIM = 128  # the head dim the tuned kernels take; also the launch-order estimate's row width
ELEMENT_DTYPES = (torch.bfloat16, torch.float16)


def heads_per_block(group: int) -> int:
    """Query heads per forward/dQ work-group (mirror of ts_attn_heads_per_block)."""
    if group % 4 == 0:
        return 4
    if group % 2 == 0:
        return 2
    return 1


def q_block_rows(hq: int, hkv: int) -> int:
    """Query rows per forward/dQ work item (mirror of ts_attn_q_block)."""
    return 32 * 4 // heads_per_block(hq // hkv)


# rows per item of the dS route's dQ pass at GQA groups that are a multiple of 4
DQ_BLOCK_ROWS = 64


def kv_block_keys(hq: int, hkv: int, head_dim: int = HEAD_DIM) -> int:
    """Keys per dK/dV work-group (mirror of ts_attn_kv_block): 64 at head dim
    256 and for GQA groups that are not a multiple of 4, else 48."""
    return 48 if (hq // hkv) % 4 == 0 and head_dim != 256 else 64


# At head dim 256 the 64-key dK/dV work items run two work-groups per CU
# (two waves of 32 keys each); a launch with fewer of them than that fills
# (512) leaves CUs half used, and the 48-key items of the key-split kernel
# (one work-group per CU, four waves of 16 keys) balance better: the branch
# shape at 16/2 heads (384 items of 64 keys) 7.06 ms against 6.54.
DKDV256_MIN_ITEMS = 512


# ---------------------------------------------------------------------------
# layout
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Run:
    source: int  # index into the call's key sources
    offset: int  # first row within the source
    length: int


@dataclass(eq=False)
class AttnLayout:
    """Integer description of one attention call (see the module docstring)."""

    q_rows: int
    hq: int
    hkv: int
    source_rows: tuple[int, ...]
    runs: tuple[Run, ...]
    seg_q: tuple[tuple[int, int], ...]  # (q_row0, q_len) per segment
    seg_spans: tuple[tuple[tuple[int, int], ...], ...]  # per segment: (run, kpos)
    seg_kv: tuple[int, ...] = field(init=False)
    _tables: dict = field(default_factory=dict, init=False, repr=False)
    _lock: threading.Lock = field(default_factory=threading.Lock, init=False, repr=False)

    def __post_init__(self):
        if self.hq <= 0 or self.hkv <= 0 or self.hq % self.hkv:
            raise ValueError(f"query heads {self.hq} are not a multiple of KV heads {self.hkv}")
        kv = []
        for s, spans in enumerate(self.seg_spans):
            pos = 0
            for run, kpos in spans:
                if not 0 <= run < len(self.runs):
                    raise ValueError(f"segment {s} names run {run} of {len(self.runs)}")
                if kpos != pos:
                    raise ValueError(f"segment {s}: spans must tile its keys in order (kpos {kpos} != {pos})")
                pos += self.runs[run].length
            kv.append(pos)
        object.__setattr__(self, "seg_kv", tuple(kv))
        if len(self.seg_q) != len(self.seg_spans):
            raise ValueError("one span list per segment")
        for s, (row0, length) in enumerate(self.seg_q):
            if length < 0 or row0 < 0 or row0 + length > self.q_rows:
                raise ValueError(f"segment {s} rows [{row0}, {row0 + length}) outside [0, {self.q_rows})")
            if length > 0 and self.seg_kv[s] < length:
                raise ValueError(
                    f"segment {s} has {length} query rows but only {self.seg_kv[s]} keys; "
                    "bottom-right causal attention needs kv_len >= q_len"
                )
        for r, run in enumerate(self.runs):
            if not 0 <= run.source < len(self.source_rows):
                raise ValueError(f"run {r} names source {run.source}")
            if run.length <= 0 or run.offset < 0 or run.offset + run.length > self.source_rows[run.source]:
                raise ValueError(f"run {r} rows outside its source")
        # the backward writes each run's dK/dV through its own rows, without
        # atomics: two runs may not share a row of a source
        by_source: dict[int, list[tuple[int, int, int]]] = {}
        for r, run in enumerate(self.runs):
            by_source.setdefault(run.source, []).append((run.offset, run.offset + run.length, r))
        for source, spans in by_source.items():
            spans.sort()
            for (a0, a1, ra), (b0, _b1, rb) in zip(spans, spans[1:]):
                if b0 < a1:
                    raise ValueError(f"runs {ra} and {rb} overlap in source {source} (rows {b0}..{a1 - 1})")
        if max([*self.seg_kv, 0]) >= 2**31 or self.q_rows >= 2**40:
            raise ValueError("attention problem too large")

    # -- work lists ---------------------------------------------------------
    def _host_tables(self, kvb: int | None = None):
        qb = q_block_rows(self.hq, self.hkv)
        segs = np.zeros(len(self.seg_q), SEG_DTYPE)
        spans, visits_of = [], [[] for _ in self.runs]
        q_items = []
        for s, ((row0, length), sp) in enumerate(zip(self.seg_q, self.seg_spans)):
            segs[s] = (row0, length, self.seg_kv[s], len(spans), len(sp))
            for run, kpos in sp:
                spans.append((run, kpos))
                visits_of[run].append((s, kpos))
            off = self.seg_kv[s] - length
            for q0 in range(0, length, qb):
                # visible keys of the block's last row: the block's cost
                last = min(q0 + qb, length) - 1
                q_items.append((-(off + last + 1), s, q0))
        visit_rows, visit0 = [], []
        for run, vis in enumerate(visits_of):
            visit0.append(len(visit_rows))
            visit_rows.extend(vis)
        # dK/dV items: every kvb-key block of every visited run; its cost is
        # the number of query rows that see its first key, over its visits
        kvb = kv_block_keys(self.hq, self.hkv) if kvb is None else kvb
        seg_len = np.array([n for _, n in self.seg_q], np.int64)
        seg_off = np.array(self.seg_kv, np.int64) - seg_len
        kv_cost, kv_run, kv_k0 = [], [], []
        for run, vis in enumerate(visits_of):
            if not vis:
                continue
            k0 = np.arange(0, self.runs[run].length, kvb, dtype=np.int64)
            seg = np.array([s for s, _ in vis], np.int64)
            kpos = np.array([kp for _, kp in vis], np.int64)
            q_len, off = seg_len[seg], seg_off[seg]
            first_row = np.maximum(0, kpos[None, :] + k0[:, None] - off[None, :])
            kv_cost.append(np.maximum(0, q_len[None, :] - first_row).sum(axis=1))
            kv_run.append(np.full(k0.shape, run, np.int64))
            kv_k0.append(k0)
        # longest cost band first, then segment and row (ORDER_BAND)
        if q_items:
            qa = np.array(q_items, np.int64).reshape(-1, 3)
            q_items = [q_items[i] for i in np.lexsort((qa[:, 2], qa[:, 1], -_cost_band(-qa[:, 0])))]
        q_work = np.array([(s, q0) for _, s, q0 in q_items], np.int32).reshape(-1, 2)
        if kv_cost:
            cost, run_of, k0_of = (np.concatenate(x) for x in (kv_cost, kv_run, kv_k0))
            order = np.lexsort((k0_of, run_of, -_cost_band(cost)))  # cost band descending, then run, then k0
            kv_work = np.stack([run_of[order], k0_of[order]], axis=1).astype(np.int32)
            kv_costs = cost[order].tolist()
        else:
            kv_work = np.zeros((0, 2), np.int32)
            kv_costs = []
        group = self.hq // self.hkv
        # rows the forward / dQ work-groups re-read: K and V of every run; the
        # dK/dV work-groups: Q and dO of every row (2-byte elements, all heads)
        kv_bytes = sum(run.length for run in self.runs) * self.hkv * HEAD_DIM * 2 * 2
        q_bytes = self.q_rows * self.hq * HEAD_DIM * 2 * 2
        q_long = _long_items([-c for c, _, _ in q_items], self.hkv * (group // heads_per_block(group)), kv_bytes)
        kv_long = _long_items(kv_costs, self.hkv, q_bytes)
        # the dS route's dQ pass over 64-row items (GQA groups that are a
        # multiple of 4): a dQ work-group then shares its K tiles between the
        # two 32-row blocks of its four heads
        dq_work, dq_long = np.zeros((0, 2), np.int32), 0
        if group % 4 == 0:
            dq_items = []
            for s_, ((_, length), kv) in enumerate(zip(self.seg_q, self.seg_kv)):
                for q0 in range(0, length, DQ_BLOCK_ROWS):
                    dq_items.append((-(kv - length + min(q0 + DQ_BLOCK_ROWS, length)), s_, q0))
            if dq_items:
                da = np.array(dq_items, np.int64).reshape(-1, 3)
                dq_items = [dq_items[i] for i in np.lexsort((da[:, 2], da[:, 1], -_cost_band(-da[:, 0])))]
                dq_work = np.array([(s_, q0) for _, s_, q0 in dq_items], np.int32).reshape(-1, 2)
                dq_long = _long_items([-c for c, _, _ in dq_items], self.hkv * (group // 4), kv_bytes)
        seg_spans = np.array(spans, REF_DTYPE) if spans else np.zeros(0, REF_DTYPE)
        run_visits = np.array(visit_rows, REF_DTYPE) if visit_rows else np.zeros(0, REF_DTYPE)
        return (segs, seg_spans, run_visits, q_work, kv_work, visit0, [len(v) for v in visits_of],
                q_long, kv_long, dq_work, dq_long)

    def device_tables(self, device: torch.device, kv_block: int | None = None):
        """Upload the layout's integer tables once per device and dK/dV item
        size (pinned, non-blocking); `kv_block` None: the head-dim-128 size."""
        kvb = kv_block_keys(self.hq, self.hkv) if kv_block is None else int(kv_block)
        key = (device.type, device.index, kvb)
        hit = self._tables.get(key)
        if hit is not None:
            return hit
        with self._lock:
            hit = self._tables.get(key)
            if hit is None:
                (segs, spans, visits, q_work, kv_work, visit0, nvisit, q_long, kv_long, dq_work,
                 dq_long) = self._host_tables(kvb)
                parts = [segs.view(np.uint8), spans.view(np.uint8), visits.view(np.uint8),
                         q_work.view(np.uint8).reshape(-1), kv_work.view(np.uint8).reshape(-1),
                         dq_work.view(np.uint8).reshape(-1)]
                offsets, total = [], 0
                for p in parts:
                    offsets.append(total)
                    total += (p.size + 255) // 256 * 256
                blob = np.zeros(max(total, 256), np.uint8)
                for o, p in zip(offsets, parts):
                    blob[o : o + p.size] = p
                host = torch.from_numpy(blob).pin_memory() if device.type == "cuda" else torch.from_numpy(blob)
                dev = host.to(device, non_blocking=True)
                base = dev.data_ptr()
                hit = {
                    "blob": dev,
                    "host": host,
                    "arrays": (segs, spans, visits, q_work, kv_work),
                    "segs": base + offsets[0],
                    "seg_spans": base + offsets[1],
                    "run_visits": base + offsets[2],
                    "q_work": base + offsets[3],
                    "kv_work": base + offsets[4],
                    "dq_work": base + offsets[5] if dq_work.shape[0] else None,
                    "n_dq_work": int(dq_work.shape[0]),
                    "n_dq_long": int(dq_long),
                    "n_q_work": int(q_work.shape[0]),
                    "n_kv_work": int(kv_work.shape[0]),
                    "visit0": visit0,
                    "nvisit": nvisit,
                    "n_q_long": q_long,
                    "n_kv_long": kv_long,
                }
                self._tables[key] = hit
        return hit

    def ds_tables(self, device: torch.device) -> dict:
        """The dS route's workspace layout (``ts_attn_ds_layout``): elements per
        head and the per-span / per-visit offsets, uploaded once per device."""
        key = ("ds", device.type, device.index)
        hit = self._tables.get(key)
        if hit is not None:
            return hit
        tabs = self.device_tables(device)
        with self._lock:
            hit = self._tables.get(key)
            if hit is None:
                segs, spans, visits, _, _ = tabs["arrays"]
                run_len = np.array([r.length for r in self.runs], np.int32)
                visit0 = np.array(tabs["visit0"], np.int32)
                nvisit = np.array(tabs["nvisit"], np.int32)
                span_ds = np.zeros(max(spans.shape[0], 1), np.int64)
                visit_ds = np.zeros(max(visits.shape[0], 1), np.int64)
                head = ctypes.c_int64(0)

                def ptr(a):
                    return a.ctypes.data if a.size else None

                lib = _lib.require_library()
                _lib.check(
                    lib.ts_attn_ds_layout(ptr(segs), len(segs), ptr(spans), spans.shape[0], ptr(run_len),
                                          len(run_len), ptr(visits), ptr(visit0), ptr(nvisit), visits.shape[0],
                                          span_ds.ctypes.data, visit_ds.ctypes.data, ctypes.byref(head)),
                    "ts_attn_ds_layout",
                )
                blob = np.concatenate([span_ds, visit_ds])
                host = torch.from_numpy(blob).pin_memory() if device.type == "cuda" else torch.from_numpy(blob)
                dev = host.to(device, non_blocking=True)
                hit = {
                    "blob": dev,
                    "host": host,
                    "head": int(head.value),
                    "span": dev.data_ptr(),
                    "visit": dev.data_ptr() + 8 * span_ds.shape[0],
                    "span_ds": span_ds[: spans.shape[0]],
                    "visit_ds": visit_ds[: visits.shape[0]],
                }
                self._tables[key] = hit
        return hit

    def kv_block_for(self, device, head_dim: int) -> int:
        """Keys per dK/dV work item at `head_dim`: ts_attn_kv_block's, except
        at head dim 256 when the 64-key items of the visited runs, over all
        KV heads, are fewer than DKDV256_MIN_ITEMS: then 48 (the key-split
        kernel)."""
        kvb = kv_block_keys(self.hq, self.hkv, head_dim)
        if head_dim == 256:
            nvisit = self.device_tables(device)["nvisit"]
            n64 = sum((run.length + 63) // 64 for run, nv in zip(self.runs, nvisit) if nv)
            if n64 * self.hkv < DKDV256_MIN_ITEMS:
                kvb = 48
        return kvb

    def problem(self, device, runs_ptr: int, scale: float, dtype: torch.dtype = torch.bfloat16,
                head_dim: int = HEAD_DIM) -> AttnProblem:
        kvb = self.kv_block_for(device, int(head_dim))
        t = self.device_tables(device, kvb)
        return AttnProblem(
            t["segs"], t["seg_spans"], runs_ptr, t["run_visits"], t["q_work"], t["kv_work"],
            t["n_q_work"], t["n_kv_work"], len(self.seg_q), len(self.runs), self.hq, self.hkv,
            int(head_dim), float(scale), q_block_rows(self.hq, self.hkv), kvb, self.q_rows,
            t["n_q_long"], t["n_kv_long"], _lib.dtype_code(dtype),
        )

    # -- reference diagnostics ---------------------------------------------
    def visible_pairs(self) -> int:
        """Exactly visible (query, key) pairs, per head: sum over segments."""
        total = 0
        for (_, t), s in zip(self.seg_q, self.seg_kv):
            total += t * (s - t) + t * (t + 1) // 2
        return total


# MI355X: work-group slots of one launch (256 CUs, one attention work-group
# each) and the last-level cache shared by the 8 XCDs
LAUNCH_SLOTS = 256
SHARED_CACHE_BYTES = 256 << 20


# Work items are launched in bands of costs within ORDER_BAND of each other
# (geometric), longest band first, and within a band by run (dK/dV) or
# segment (forward, dQ) and position: neighbours in the list, which the
# launch order places on one XCD together, then read the same rows and share
# its L2, while the longest-first order that keeps the end of the launch
# short changes by at most ORDER_BAND.  (C4: dK/dV 34.3 -> 32.4 ms, forward
# 11.85 -> 11.62 ms, dQ 10.7 -> 10.0 ms; C2 within noise.)
ORDER_BAND = 0.05


def _cost_band(cost: np.ndarray) -> np.ndarray:
    """Index of each cost's geometric band of width ORDER_BAND (higher for larger costs)."""
    return np.floor(np.log(np.maximum(cost, 1)) / np.log(1.0 + ORDER_BAND)).astype(np.int64)


def _long_items(costs: Sequence[int], heads: int, reread_bytes: int, slots: int = LAUNCH_SLOTS) -> int:
    """How many of the (descending) ``costs`` run item-major at the head of the
    launch (ts_attn_problem.n_*_long).

    When the rows the work-groups re-read (``reread_bytes``, all heads) fit in
    half the shared last-level cache, every item does: each XCD then serves
    fixed heads and keeps their rows in its L2 while the shared cache holds
    the rest.  Otherwise only the items long enough to stretch the end of the
    launch when started late -- a quarter or more of a slot's average share
    of the whole launch (``heads`` copies of every item) -- and the rest run
    head by head, all XCDs streaming one head's rows through the shared cache.
    """
    if reread_bytes <= SHARED_CACHE_BYTES // 2:
        return len(costs)
    total = sum(costs) * heads
    if not costs or total == 0:
        return 0
    threshold = 0.25 * total / slots
    n = 0
    while n < len(costs) and costs[n] >= threshold:
        n += 1
    return n


def _check_rows_tensor(t: torch.Tensor, name: str, heads: int, head_dim: int, max_row_stride: int = 1 << 24) -> None:
    if t.dim() != 3 or t.shape[1] != heads or t.shape[2] != head_dim:
        raise ValueError(f"{name} must be [rows, {heads}, {head_dim}], got {tuple(t.shape)}")
    if t.stride(2) != 1 or t.stride(0) % 8 or t.stride(1) % 8 or t.data_ptr() % 16:
        raise ValueError(f"{name} needs a contiguous head dim, 16-byte alignment and 8-element strides")
    if t.stride(0) >= max_row_stride:
        # the kernels address a tile's rows with 32-bit byte offsets
        raise ValueError(f"{name} row stride {t.stride(0)} must be below {max_row_stride} elements")


def _rows(t: torch.Tensor) -> AttnRows:
    return AttnRows(t.data_ptr(), t.stride(0), t.stride(1))


def _run_table(layout: AttnLayout, keys, values, dkeys=None, dvalues=None) -> torch.Tensor:
    visit = layout.device_tables(keys[0].device)
    table = np.zeros(len(layout.runs), RUN_DTYPE)
    esz = 2
    for r, run in enumerate(layout.runs):
        k, v = keys[run.source], values[run.source]
        row = table[r]
        row["k"] = k.data_ptr() + run.offset * k.stride(0) * esz
        row["v"] = v.data_ptr() + run.offset * v.stride(0) * esz
        row["k_row_stride"], row["k_head_stride"] = k.stride(0), k.stride(1)
        row["v_row_stride"], row["v_head_stride"] = v.stride(0), v.stride(1)
        if dkeys is not None:
            dk, dv = dkeys[run.source], dvalues[run.source]
            row["dk"] = dk.data_ptr() + run.offset * dk.stride(0) * esz
            row["dv"] = dv.data_ptr() + run.offset * dv.stride(0) * esz
            row["dk_row_stride"], row["dk_head_stride"] = dk.stride(0), dk.stride(1)
            row["dv_row_stride"], row["dv_head_stride"] = dv.stride(0), dv.stride(1)
        row["len"] = run.length
        row["visit0"] = visit["visit0"][r]
        row["nvisit"] = visit["nvisit"][r]
    host = torch.from_numpy(table.view(np.uint8)).pin_memory()
    return host.to(keys[0].device, non_blocking=True), host


def check_tables(layout: AttnLayout, problem: AttnProblem, run_table: np.ndarray | torch.Tensor,
                 device: torch.device) -> None:
    """Check the layout's tables for ``device`` and one call's run table on the
    host (ts_attn_check_tables) before the kernels read their device copies:
    spans tile every segment's keys, every visit is a span of its segment,
    the work lists hold every row and key block once, K/V/dK/dV addresses are
    aligned.  Raises RuntimeError naming the first inconsistency."""
    segs, spans, visits, q_work, kv_work = layout.device_tables(device, problem.kv_block)["arrays"]
    runs = run_table.numpy() if isinstance(run_table, torch.Tensor) else run_table
    runs = np.ascontiguousarray(runs).view(np.uint8)
    if runs.size != len(layout.runs) * RUN_DTYPE.itemsize:
        raise ValueError(f"run table holds {runs.size} bytes, expected {len(layout.runs)} runs")
    arrays = (segs, spans, runs, visits, q_work, kv_work)
    segs_p, spans_p, runs_p, visits_p, q_p, kv_p = (a.ctypes.data if a.size else None for a in arrays)
    lib = _lib.require_library()
    _lib.check(
        lib.ts_attn_check_tables(ctypes.byref(problem), segs_p, spans_p, spans.shape[0], runs_p, visits_p,
                                 visits.shape[0], q_p, kv_p),
        f"attention tables (rows={layout.q_rows}, segments={len(layout.seg_q)}, runs={len(layout.runs)})",
    )


def _validate_call(layout: AttnLayout, query: torch.Tensor, keys, values) -> None:
    if not query.is_cuda:
        raise RuntimeError("thundersync_amd attention runs on the GPU only; got a CPU tensor")
    if query.dtype not in ELEMENT_DTYPES:
        raise TypeError(f"thundersync_amd attention takes bf16 or fp16, got {query.dtype}")
    head_dim = query.shape[-1] if query.dim() == 3 else -1
    if head_dim not in HEAD_DIMS:
        raise ValueError(f"thundersync_amd attention takes head dims 1..{MAX_HEAD_DIM} (kernels at {HEAD_DIMS}), "
                         f"got query {tuple(query.shape)}")
    _check_rows_tensor(query, "query", layout.hq, head_dim)
    if query.shape[0] != layout.q_rows:
        raise ValueError(f"query has {query.shape[0]} rows, layout {layout.q_rows}")
    if len(keys) != len(layout.source_rows) or len(values) != len(layout.source_rows):
        raise ValueError("one K and one V tensor per key source")
    for i, (k, v) in enumerate(zip(keys, values)):
        for name, t in (("key", k), ("value", v)):
            if t.device != query.device or t.dtype != query.dtype:
                raise ValueError(f"{name} source {i} must be {query.dtype} on {query.device}")
            _check_rows_tensor(t, f"{name} source {i}", layout.hkv, head_dim)
            if t.shape[0] != layout.source_rows[i]:
                raise ValueError(f"{name} source {i} has {t.shape[0]} rows, layout {layout.source_rows[i]}")


# dS workspace (bytes) the backward may allocate for the dS route (dK/dV
# kernels store dS, dQ = dS K from it; about 2 bytes per visible pair and
# head): up to DS_MAX_BYTES, and a workspace above it when it fits in
# DS_FREE_FRACTION of the memory the device can still supply (an MI355X holds
# 288 GB; the reference's 16-trajectory retained-chunk pack needs ~52 GB);
# never more than DS_AVAILABLE_FRACTION of that memory, so a device that is
# nearly full takes the route over fewer KV heads, or not at all, instead of
# failing inside the backward.  The memory the device can supply is its free
# memory plus what torch's allocator holds unused.  A problem above the cap
# runs the route over groups of KV heads, as many per call as fit (KV heads
# are independent: their query heads, dS and gradients do not mix, and the
# grouped calls give the one-call gradients bit for bit); one whose single KV
# head does not fit, one whose workspace allocation fails all the same, or
# any under THUNDERSYNC_ATTN_DS=off, runs the route that recomputes S and dP
# in the dQ kernel.
DS_MAX_BYTES = 16 << 30
DS_FREE_FRACTION = 0.25
DS_AVAILABLE_FRACTION = 0.5
DS_ENV = "THUNDERSYNC_ATTN_DS"


def _device_free_bytes(device: torch.device) -> int:
    """Memory `device` can still supply in bytes: free device memory plus the
    allocator's reserved but unallocated bytes (0 for a host device)."""
    if device.type != "cuda":
        return 0
    free, _total = torch.cuda.mem_get_info(device)
    cached = torch.cuda.memory_reserved(device) - torch.cuda.memory_allocated(device)
    return int(free) + max(int(cached), 0)


def _ds_route(layout: AttnLayout, query: torch.Tensor, lib):
    """(workspace tables, KV heads per call) when this backward takes the dS
    route, else None."""
    if os.environ.get(DS_ENV, "auto").strip().lower() == "off" or DS_MAX_BYTES <= 0:
        return None
    group = layout.hq // layout.hkv
    if not lib.ts_attn_ds_route(query.shape[2], group):
        return None
    tabs = layout.ds_tables(query.device)
    # a call over n KV heads needs (n * group * head + 512) elements: every
    # query head's part, then the sink block
    per_kv_head = group * max(tabs["head"], 1)
    available = _device_free_bytes(query.device)
    cap = DS_MAX_BYTES
    if (layout.hkv * per_kv_head + 512) * 2 > cap and DS_FREE_FRACTION > 0:
        cap = max(cap, int(available * DS_FREE_FRACTION))
    cap = min(cap, int(available * DS_AVAILABLE_FRACTION))
    kv_heads = min(layout.hkv, (cap // 2 - 512) // per_kv_head)
    if kv_heads < 1:
        return None
    return tabs, kv_heads


def _head_rows(rows: AttnRows, first_head: int) -> AttnRows:
    """A rows view that starts at head `first_head` (2-byte elements)."""
    return AttnRows(rows.ptr + first_head * rows.head_stride * 2, rows.row_stride, rows.head_stride)


def _head_runs(host: torch.Tensor, first_kv_head: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """A copy of a run table whose K/V/dK/dV addresses start at KV head `first_kv_head`."""
    table = host.numpy().view(RUN_DTYPE).copy()
    for name in ("k", "v", "dk", "dv"):
        live = table[name] != 0
        table[name][live] += (first_kv_head * table[f"{name}_head_stride"][live] * 2).astype(np.uint64)
    sub = torch.from_numpy(table.view(np.uint8)).pin_memory() if device.type == "cuda" else torch.from_numpy(
        table.view(np.uint8))
    return sub.to(device, non_blocking=True), sub


class _Attention(torch.autograd.Function):
    """out, lse = attention over `layout`; grads to query and every key source."""

    @staticmethod
    def forward(ctx, query, layout, scale, n_sources, *kv):
        keys, values = list(kv[:n_sources]), list(kv[n_sources:])
        _validate_call(layout, query, keys, values)
        lib = _lib.require_library()
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
        lse = torch.empty(layout.hq, max(layout.q_rows, 1), dtype=torch.float32, device=query.device)
        runs, host = _run_table(layout, keys, values)
        problem = layout.problem(query.device, runs.data_ptr(), scale, query.dtype, query.shape[2])
        check_tables(layout, problem, host, query.device)
        with operator_range("hip_attention_forward", rows=layout.q_rows, segments=len(layout.seg_q)):
            _lib.check(
                lib.ts_attn_fwd(ctypes.byref(problem), _rows(query), _rows(out), lse.data_ptr(),
                                lse.shape[1], _lib.stream_of(query)),
                f"ts_attn_fwd(rows={layout.q_rows}, hq={layout.hq}, hkv={layout.hkv})",
            )
        count_attention_path(HIP_PATH)
        ctx.layout, ctx.scale, ctx.n_sources = layout, scale, n_sources
        ctx.keep = (runs, host)
        ctx.save_for_backward(query, out, lse, *kv)
        ctx.mark_non_differentiable(lse)
        ctx.set_materialize_grads(False)  # no zero-filled gradient for lse
        return out, lse

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dout, _dlse):
        query, out, lse, *kv = ctx.saved_tensors
        layout, n = ctx.layout, ctx.n_sources
        keys, values = kv[:n], kv[n:]
        lib = _lib.require_library()
        if dout is None:
            dout = torch.zeros_like(out)
        dout = dout.contiguous() if dout.stride(2) != 1 or dout.stride(0) % 8 or dout.stride(1) % 8 else dout
        # dQ in the query's own layout where it is dense (a [1, Hq, T, D] query
        # seen as rows gets its gradient without a copy into that layout)
        dq = torch.empty_like(query)
        if dq.stride(2) != 1 or dq.stride(0) % 8 or dq.stride(1) % 8:
            dq = torch.empty(query.shape, dtype=query.dtype, device=query.device)
        covered = sum(t for _, t in layout.seg_q)
        if covered != layout.q_rows:
            dq.zero_()
        dkeys = [torch.empty(k.shape, dtype=k.dtype, device=k.device) for k in keys]
        dvalues = [torch.empty(v.shape, dtype=v.dtype, device=v.device) for v in values]
        # rows of a source that no run covers, or runs nobody reads, get zeros
        visit = layout.device_tables(query.device)
        covered_rows = [0] * n
        for r, run in enumerate(layout.runs):
            if visit["nvisit"][r]:
                covered_rows[run.source] += run.length
        for i in range(n):
            if covered_rows[i] != layout.source_rows[i]:
                dkeys[i].zero_()
                dvalues[i].zero_()
        runs, host = _run_table(layout, keys, values, dkeys, dvalues)
        rowstats = torch.empty(layout.hq, max(layout.q_rows, 1), 2, dtype=torch.float32, device=query.device)
        problem = layout.problem(query.device, runs.data_ptr(), ctx.scale, query.dtype, query.shape[2])
        check_tables(layout, problem, host, query.device)
        ds = _ds_route(layout, query, lib)
        if ds is not None:
            tabs, kv_heads = ds
            group = layout.hq // layout.hkv
            try:
                work = torch.empty(kv_heads * group * tabs["head"] + 512, dtype=query.dtype,
                                   device=query.device)
            except torch.cuda.OutOfMemoryError:
                ds = None
        with operator_range("hip_attention_backward", rows=layout.q_rows, segments=len(layout.seg_q),
                            ds_route=ds is not None):
            if ds is None:
                _lib.check(
                    lib.ts_attn_bwd(ctypes.byref(problem), _rows(query), _rows(out), _rows(dout),
                                    lse.data_ptr(), lse.shape[1], rowstats.data_ptr(), _rows(dq),
                                    _lib.stream_of(query)),
                    f"ts_attn_bwd(rows={layout.q_rows}, hq={layout.hq}, hkv={layout.hkv})",
                )
            else:
                rows = [_rows(t) for t in (query, out, dout, dq)]
                keep = []
                # the dQ pass's 64-row list where it applies (head dim 128, groups of 4)
                dq_list, n_dq, n_dq_long = None, 0, 0
                if query.shape[2] == HEAD_DIM and visit["dq_work"] is not None:
                    dq_list, n_dq, n_dq_long = visit["dq_work"], visit["n_dq_work"], visit["n_dq_long"]
                for hk0 in range(0, layout.hkv, kv_heads):
                    n, h0 = min(kv_heads, layout.hkv - hk0), hk0 * group
                    sub = problem
                    if n != layout.hkv:  # KV heads hk0 .. hk0 + n - 1 and their query heads
                        sub_runs, sub_host = _head_runs(host, hk0, query.device)
                        keep.append((sub_runs, sub_host))
                        sub = AttnProblem.from_buffer_copy(problem)
                        sub.hq, sub.hkv, sub.runs = n * group, n, sub_runs.data_ptr()
                        check_tables(layout, sub, sub_host, query.device)
                    q_r, o_r, do_r, dq_r = (_head_rows(r, h0) for r in rows)
                    _lib.check(
                        lib.ts_attn_bwd_ds(ctypes.byref(sub), q_r, o_r, do_r, lse.data_ptr() + h0 * lse.shape[1] * 4,
                                           lse.shape[1], rowstats.data_ptr() + h0 * lse.shape[1] * 8, dq_r,
                                           tabs["span"], tabs["visit"], tabs["head"], work.data_ptr(),
                                           work.numel() * 2, dq_list, n_dq, n_dq_long, _lib.stream_of(query)),
                        f"ts_attn_bwd_ds(rows={layout.q_rows}, hq={layout.hq}, hkv={layout.hkv}, heads from {h0})",
                    )
                ctx.keep_bwd_heads = keep
                del work
        count_attention_path(HIP_BACKWARD_PATH)
        ctx.keep_bwd = (runs, host)
        return (dq, None, None, None, *dkeys, *dvalues)


def kernel_head_dim(head_dim: int) -> int | None:
    """The kernel head dim that runs `head_dim`: itself when the kernels are
    built for it, else the next larger one (for 1 <= head_dim <= 256), None
    above 256.  Zero columns appended to Q and K change no score and zero
    columns of V only add output columns, so the padded call's output and
    gradients restricted to the first `head_dim` columns are the unpadded
    ones; the caller's scale is used as given."""
    if head_dim < 1:
        return None
    for d in HEAD_DIMS:
        if head_dim <= d:
            return d
    return None


def attention(query: torch.Tensor, layout: AttnLayout, keys: Sequence[torch.Tensor],
              values: Sequence[torch.Tensor], scale: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Core op: query ``[R, Hq, D]`` bf16 or fp16 -> (out ``[R, Hq, D]``, lse ``[Hq, R]`` fp32).

    A head dim the kernels are not built for (any other D up to 256) runs at
    :func:`kernel_head_dim` over zero-padded copies of Q, K and V; autograd
    takes the gradients back through the padding."""
    d = query.shape[-1] if query.dim() == 3 else -1
    dk = kernel_head_dim(d)
    if dk is not None and dk != d:
        def pad(t):
            return torch.nn.functional.pad(t, (0, dk - t.shape[-1]))
        out, lse = _Attention.apply(pad(query), layout, float(scale), len(keys), *(pad(k) for k in keys),
                                    *(pad(v) for v in values))
        return out[..., :d], lse
    return _Attention.apply(query, layout, float(scale), len(keys), *keys, *values)


# ---------------------------------------------------------------------------
# layouts for the reference's call shapes
# ---------------------------------------------------------------------------
def _dedupe(tensors: Sequence[torch.Tensor]):
    """Distinct tensors (by identity) and, per input position, its source index."""
    sources, index, where = [], {}, []
    for t in tensors:
        key = id(t)
        if key not in index:
            index[key] = len(sources)
            sources.append(t)
        where.append(index[key])
    return sources, where


def chain_layout(query_len: int, chunk_lengths: Sequence[int], hq: int, hkv: int) -> AttnLayout:
    """One segment of `query_len` rows over the concatenation of chunks."""
    runs = tuple(Run(i, 0, n) for i, n in enumerate(chunk_lengths) if n > 0)
    spans, pos = [], 0
    run_index = 0
    for i, n in enumerate(chunk_lengths):
        if n > 0:
            spans.append((run_index, pos))
            run_index += 1
            pos += n
    return AttnLayout(
        q_rows=query_len, hq=hq, hkv=hkv, source_rows=tuple(chunk_lengths), runs=runs,
        seg_q=((0, query_len),), seg_spans=(tuple(spans),),
    )


def _query_rows(query: torch.Tensor) -> torch.Tensor:
    """``[1, Hq, T, D]`` (any strides) -> ``[T, Hq, D]`` view."""
    if query.dim() != 4 or query.shape[0] != 1:
        raise ValueError(f"query must be [1, Hq, T, D], got {tuple(query.shape)}")
    # squeeze, not select: the gradient of a select is a zero-filled copy
    return query.squeeze(0).transpose(0, 1)


def _as_rows(t: torch.Tensor) -> torch.Tensor:
    """A [rows, heads, D] view usable by the kernels (copy only if it must)."""
    if t.stride(2) == 1 and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0 and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def causal_attention(query: torch.Tensor, ks: Sequence[torch.Tensor], vs: Sequence[torch.Tensor],
                     scale: float) -> torch.Tensor:
    """Backend callable ``(query [1,Hq,T,D], ks, vs, scale) -> [1,Hq,T,D]``.

    ``ks``/``vs`` are chunk lists ``[S_c, Hkv, D]`` in chronological order;
    query row i sees keys ``0 .. S - T + i`` of their concatenation, which is
    never materialised (engine/streaming.py:1080-1162).
    """
    q = _as_rows(_query_rows(query))
    keys, kw = _dedupe(ks)
    values, vw = _dedupe(vs)
    if kw != vw or len(keys) != len(ks):
        # distinct chunk objects per position keep one run per chunk
        keys, values = list(ks), list(vs)
    keys = [_as_rows(k) for k in keys]
    values = [_as_rows(v) for v in values]
    layout = chain_layout(q.shape[0], [k.shape[0] for k in keys], q.shape[1], keys[0].shape[1])
    out, _ = attention(q, layout, keys, values, scale)
    return out.transpose(0, 1).unsqueeze(0)


class ChunkedCausalAttention(torch.autograd.Function):
    """``apply(query, scale, n_chunks, keep_state, backend, *ks, *vs)``.

    Argument order and meaning of ``_ChunkedCausalSDPA`` (engine/streaming.py:
    1314-1423): bottom-right-causal attention of ``query [1, Hq, T, D]`` over
    the chunk lists as one op that keeps only references to the per-chunk K/V
    (never a concatenated copy) and returns one dK/dV per chunk in input order.

    * ``backend`` ``"auto"`` or ``"cudnn"`` (the reference's built-in names):
      the HIP kernels.  The op keeps the query, its output and log-sum-exp --
      what the reference's saved-state mode keeps -- and its backward runs
      the HIP backward on them, whatever ``keep_state`` says (the reference's
      other mode re-runs the forward to reach the same numbers; the HIP
      forward is deterministic, so keeping them is equivalent).
    * a callable ``backend(query, ks, vs, scale)``: called as the reference
      calls it (:1094-1095), and differentiated by re-running it under
      autograd in the backward (:1384-1399).
    * any other name raises ``ValueError`` (:1096-1097).
    """

    @staticmethod
    def forward(ctx, query, scale, n_chunks, keep_state, backend, *chunks):
        ks, vs = list(chunks[:n_chunks]), list(chunks[n_chunks:])
        ctx.n_chunks, ctx.scale, ctx.backend = n_chunks, scale, backend
        if callable(backend):
            ctx.graph = None
            ctx.save_for_backward(query, *chunks)
            return backend(query, ks, vs, scale)
        if backend not in ("auto", "cudnn"):
            raise ValueError(f"unknown source attention backend: {backend!r}")
        with torch.enable_grad():
            leaves = [c.detach().requires_grad_(c.requires_grad) for c in chunks]
            q = query.detach().requires_grad_(query.requires_grad)
            out = causal_attention(q, leaves[:n_chunks], leaves[n_chunks:], scale)
        ctx.graph = (q, leaves, out)
        return out.detach()

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        need = ctx.needs_input_grad
        n = ctx.n_chunks
        if ctx.graph is None:
            query, *chunks = ctx.saved_tensors
            q = query.detach().requires_grad_(True)
            leaves = [c.detach().requires_grad_(True) for c in chunks]
            with torch.enable_grad():
                out = ctx.backend(q, leaves[:n], leaves[n:], ctx.scale)
            grads = torch.autograd.grad(out, [q, *leaves], grad_out, allow_unused=True)
            dq, rest = grads[0], list(grads[1:])
        else:
            q, leaves, out = ctx.graph
            inputs = [t for t in (q, *leaves) if t.requires_grad]
            grads = torch.autograd.grad(out, inputs, grad_out, allow_unused=True) if inputs else []
            it = iter(grads)
            dq = next(it) if q.requires_grad else None
            rest = [next(it) if c.requires_grad else None for c in leaves]
        return (
            dq if need[0] else None, None, None, None, None,
            *(g if need[5 + i] else None for i, g in enumerate(rest)),
        )


@dataclass(eq=False)
class PackLayout:
    """Where each segment of a plain turn pack sits (engine/streaming.py:1613-1650).

    ``lengths``: query rows per segment; ``prefixes``: ancestor tokens per
    segment; ``counts``: ancestor chunks per segment.  ``cu_lengths`` and
    ``cu_prefixes`` are the int32 cumulative sums ``[0, *accumulate(...)]``.
    The op's ancestor inputs are grouped by segment, LAST segment first.
    """

    lengths: list[int]
    prefixes: list[int]
    counts: list[int]
    cu_lengths: torch.Tensor
    cu_prefixes: torch.Tensor
    counted: bool = True

    def inputs(self, ancestors):
        ks = [c for ks, _vs in reversed(ancestors) for c in ks]
        vs = [c for _ks, vs in reversed(ancestors) for c in vs]
        return ks + vs

    def by_segment(self, chunks):
        grouped, offset = [], 0
        for count in reversed(self.counts):
            grouped.append(list(chunks[offset : offset + count]))
            offset += count
        return grouped[::-1]


def pack_layout(lengths: Sequence[int], ancestors, device=None) -> PackLayout:
    """Build a PackLayout from per-segment lengths and ancestor chunk lists."""
    from itertools import accumulate

    prefixes = [sum(c.shape[0] for c in ks) for ks, _vs in ancestors]
    counts = [len(ks) for ks, _vs in ancestors]
    cu_l = torch.tensor([0, *accumulate(lengths)], dtype=torch.int32)
    cu_p = torch.tensor([0, *accumulate(prefixes)], dtype=torch.int32)
    if device is not None and torch.device(device).type == "cuda":
        cu_l = cu_l.pin_memory().to(device, non_blocking=True)
        cu_p = cu_p.pin_memory().to(device, non_blocking=True)
    return PackLayout(list(lengths), prefixes, counts, cu_l, cu_p)


class PackedAttention(torch.autograd.Function):
    """``apply(query, key, value, scale, layout, *ancestors)``, as _PackedFlashSplit.

    ``query [1, Hq, sum(T), D]``, the pack's own ``key``/``value`` ``[sum(T),
    Hkv, D]``, then the ancestor chunks in ``PackLayout.inputs`` order.  Each
    segment attends to its ancestors (fully) then its own rows (causally);
    one forward and one backward launch serve the whole pack.  A chunk object
    passed for several segments (the shared prompt) is one key run visited
    by each of them, so its gradient is summed inside the kernel.
    """

    @staticmethod
    def forward(ctx, query, key, value, scale, layout, *ancestors):
        total = sum(layout.counts)
        a_keys = layout.by_segment(ancestors[:total])
        a_vals = layout.by_segment(ancestors[total:])
        q = _as_rows(_query_rows(query))
        own_k, own_v = _as_rows(key), _as_rows(value)
        srcs_k, srcs_v, src_index = [own_k], [own_v], {}
        runs: list[Run] = []
        seg_q, seg_spans = [], []
        row0 = 0
        # own-K/V runs, one per segment (source 0)
        own_runs = []
        for length in layout.lengths:
            own_runs.append(len(runs))
            runs.append(Run(0, row0, length))
            row0 += length
        chunk_run = {}
        for s, (length, ks, vs) in enumerate(zip(layout.lengths, a_keys, a_vals)):
            spans, pos = [], 0
            for kc, vc in zip(ks, vs):
                if kc.shape[0] == 0:
                    continue
                ident = (id(kc), id(vc))
                if ident not in chunk_run:
                    if ident not in src_index:
                        src_index[ident] = len(srcs_k)
                        srcs_k.append(_as_rows(kc))
                        srcs_v.append(_as_rows(vc))
                    chunk_run[ident] = len(runs)
                    runs.append(Run(src_index[ident], 0, kc.shape[0]))
                spans.append((chunk_run[ident], pos))
                pos += kc.shape[0]
            if length > 0:
                spans.append((own_runs[s], pos))
            seg_q.append((sum(layout.lengths[:s]), length))
            seg_spans.append(tuple(spans))
        att_layout = AttnLayout(
            q_rows=q.shape[0], hq=q.shape[1], hkv=own_k.shape[1],
            source_rows=tuple(t.shape[0] for t in srcs_k), runs=tuple(runs),
            seg_q=tuple(seg_q), seg_spans=tuple(seg_spans),
        )
        with torch.enable_grad():
            qd = q.detach().requires_grad_(query.requires_grad)
            kd = [t.detach().requires_grad_(True) for t in srcs_k]
            vd = [t.detach().requires_grad_(True) for t in srcs_v]
            out, _ = attention(qd, att_layout, kd, vd, scale)
        ctx.graph = (qd, kd, vd, out, src_index, layout, a_keys, a_vals)
        return out.detach().transpose(0, 1).unsqueeze(0)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        qd, kd, vd, out, src_index, layout, a_keys, a_vals = ctx.graph
        g = grad_out[0].transpose(0, 1)
        inputs = ([qd] if qd.requires_grad else []) + kd + vd
        grads = torch.autograd.grad(out, inputs, g)
        it = iter(grads)
        dq = next(it).transpose(0, 1).unsqueeze(0) if qd.requires_grad else None
        dks = [next(it) for _ in kd]
        dvs = [next(it) for _ in vd]
        # ancestor grads in input order; a chunk object appearing several
        # times receives its summed gradient once (autograd adds per input)
        seen = set()
        anc_k, anc_v = [], []
        for ks, vs in zip(reversed(a_keys), reversed(a_vals)):
            for kc, vc in zip(ks, vs):
                ident = (id(kc), id(vc))
                if kc.shape[0] == 0:
                    anc_k.append(torch.zeros_like(kc))
                    anc_v.append(torch.zeros_like(vc))
                elif ident in seen:
                    anc_k.append(None)
                    anc_v.append(None)
                else:
                    seen.add(ident)
                    anc_k.append(dks[src_index[ident]])
                    anc_v.append(dvs[src_index[ident]])
        return (dq, dks[0], dvs[0], None, None, *anc_k, *anc_v)


def _ragged_layout(lengths: Sequence[int], key_rows: Sequence[int], hq: int, hkv: int) -> AttnLayout:
    """Segment i: ``lengths[i]`` packed query rows over key source i alone."""
    runs = tuple(Run(i, 0, n) for i, n in enumerate(key_rows))
    seg_q, row0 = [], 0
    for n in lengths:
        seg_q.append((row0, n))
        row0 += n
    return AttnLayout(
        q_rows=row0, hq=hq, hkv=hkv, source_rows=tuple(key_rows), runs=runs,
        seg_q=tuple(seg_q), seg_spans=tuple(((i, 0),) for i in range(len(key_rows))),
    )


def ragged_causal_attention(queries, keys, values, scale):
    """``_ragged_causal_sdpa`` (engine/streaming.py:1165-1226): per segment
    ``[1,Hq,T_i,D]`` over its own ``[S_i,Hkv,D]``, bottom-right causal, all
    segments in one launch.  Differentiable (one backward launch)."""
    if not queries:
        return []
    q_rows = [_as_rows(_query_rows(q)) for q in queries]
    lengths = [q.shape[0] for q in q_rows]
    packed = torch.cat(q_rows, 0)
    srcs_k = [_as_rows(k) for k in keys]
    srcs_v = [_as_rows(v) for v in values]
    layout = _ragged_layout(lengths, [k.shape[0] for k in srcs_k], packed.shape[1], srcs_k[0].shape[1])
    out, _ = attention(packed, layout, srcs_k, srcs_v, scale)
    return [piece.transpose(0, 1).unsqueeze(0) for piece in out.split(lengths, 0)]


class RaggedAttention(torch.autograd.Function):
    """``apply(scale, n_segments, *queries, *keys, *values)`` -> one output per
    segment, as ``_RaggedAttentionIndependentVJP`` (engine/streaming.py:
    1253-1297).  The reference runs the cohort through one varlen flash call
    and recomputes each segment with ``_causal_sdpa`` in its backward; here
    the forward is one HIP launch for the cohort and the backward one HIP
    backward launch over the saved output and log-sum-exp, which gives every
    segment its own independent VJP (segments share no keys)."""

    @staticmethod
    def forward(ctx, scale, n_segments, *tensors):
        queries = list(tensors[:n_segments])
        keys = list(tensors[n_segments : 2 * n_segments])
        values = list(tensors[2 * n_segments :])
        with torch.enable_grad():
            qs = [q.detach().requires_grad_(q.requires_grad) for q in queries]
            kk = [k.detach().requires_grad_(k.requires_grad) for k in keys]
            vv = [v.detach().requires_grad_(v.requires_grad) for v in values]
            outs = ragged_causal_attention(qs, kk, vv, scale)
        ctx.graph = (qs + kk + vv, outs)
        return tuple(o.detach() for o in outs)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *grad_outputs):
        leaves, outs = ctx.graph
        inputs = [t for t in leaves if t.requires_grad]
        grads = torch.autograd.grad(outs, inputs, grad_outputs, allow_unused=True) if inputs else []
        it = iter(grads)
        return (None, None, *(next(it) if t.requires_grad else None for t in leaves))


# ---------------------------------------------------------------------------
# retained chunks
# ---------------------------------------------------------------------------
def retained_chunk_layout(q_rows: int, chunk_rows: Sequence[int], chunks: Sequence[tuple[int, int, Sequence[int]]],
                          hq: int, hkv: int) -> AttnLayout:
    """Query chunks over graph-retained per-chunk K/V, all in one launch.

    ``chunk_rows[i]`` is the row count of retained chunk ``i`` (one K and one
    V tensor each); ``chunks`` lists every query chunk as ``(q_row0, q_len,
    path)`` where ``path`` names, in key order, the retained chunks the query
    chunk reads -- the prompt's chunks, the earlier chunks of its trajectory
    and its own chunk last.  Each query chunk is the bottom-right-causal call
    ``_ChunkedCausalSDPA`` makes per chunk (engine/streaming.py:1314-1354);
    the retained tensors are read in place, never concatenated.
    """
    runs = tuple(Run(i, 0, n) for i, n in enumerate(chunk_rows))
    seg_q, seg_spans = [], []
    for row0, length, path in chunks:
        spans, pos = [], 0
        for c in path:
            if not 0 <= c < len(runs):
                raise ValueError(f"query chunk at row {row0} names retained chunk {c} of {len(runs)}")
            spans.append((c, pos))
            pos += runs[c].length
        seg_q.append((row0, length))
        seg_spans.append(tuple(spans))
    return AttnLayout(q_rows=q_rows, hq=hq, hkv=hkv, source_rows=tuple(chunk_rows), runs=runs,
                      seg_q=tuple(seg_q), seg_spans=tuple(seg_spans))


def retained_chunk_attention(query: torch.Tensor, ks: Sequence[torch.Tensor], vs: Sequence[torch.Tensor],
                             layout: AttnLayout, scale: float) -> torch.Tensor:
    """``query`` ``[R, Hq, D]`` over retained chunks ``ks``/``vs`` (each
    ``[S_c, Hkv, D]``) as described by :func:`retained_chunk_layout`;
    differentiable wrt the query and every retained chunk."""
    out, _ = attention(_as_rows(query), layout, [_as_rows(k) for k in ks], [_as_rows(v) for v in vs], scale)
    return out


# ---------------------------------------------------------------------------
# forest
# ---------------------------------------------------------------------------
def forest_layout(plan, hq: int, hkv: int) -> AttnLayout:
    """Segments = non-empty nodes, runs = node ranges of the one K/V tensor.

    ``plan`` is an ExecutionPlan (engine/plan.py:41-73) or anything with
    ``node_start``, ``node_end`` (per node) and ``key_ranges`` (per node:
    ancestor spans then the node's own span, engine/plan.py:248-256).
    """
    cached = getattr(plan, "_thundersync_hip_layouts", None)
    if cached is not None and (hq, hkv) in cached:
        return cached[(hq, hkv)]
    starts = [int(x) for x in plan.node_start.tolist()]
    ends = [int(x) for x in plan.node_end.tolist()]
    p = int(plan.n_physical) if hasattr(plan, "n_physical") else max(ends, default=0)
    run_of_start = {}
    runs = []
    for n, (s, e) in enumerate(zip(starts, ends)):
        if e > s:
            run_of_start[(s, e)] = len(runs)
            runs.append(Run(0, s, e - s))
    order = sorted((n for n in range(len(starts)) if ends[n] > starts[n]), key=lambda n: starts[n])
    seg_q, seg_spans = [], []
    for n in order:
        spans, pos = [], 0
        for s, e in plan.key_ranges[n]:
            if e <= s:
                continue
            if (s, e) not in run_of_start:
                raise ValueError(f"key range ({s}, {e}) of node {n} is not a node range")
            spans.append((run_of_start[(s, e)], pos))
            pos += e - s
        seg_q.append((starts[n], ends[n] - starts[n]))
        seg_spans.append(tuple(spans))
    layout = AttnLayout(
        q_rows=p, hq=hq, hkv=hkv, source_rows=(p,), runs=tuple(runs),
        seg_q=tuple(seg_q), seg_spans=tuple(seg_spans),
    )
    try:
        if cached is None:
            cached = {}
            object.__setattr__(plan, "_thundersync_hip_layouts", cached)
        cached[(hq, hkv)] = layout
    except (AttributeError, TypeError):
        pass
    return layout


def forest_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, plan, *, scale: float | None = None):
    """Attention over a segment forest on the physical stream (engine/attention.py:186-231).

    ``q`` ``[P, Hq, D]``, ``k``/``v`` ``[P, Hkv, D]``; returns ``[P, Hq, D]``.
    Every node attends to its ancestors in full and to itself causally, in
    one launch per direction; no mask and no ancestor concatenation.
    """
    scale = scale if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    if q.shape[1] % k.shape[1]:
        raise ValueError(f"query heads {q.shape[1]} are not divisible by KV heads {k.shape[1]}")
    layout = forest_layout(plan, q.shape[1], k.shape[1])
    out, _ = attention(_as_rows(q), layout, [_as_rows(k)], [_as_rows(v)], scale)
    return out


# ---------------------------------------------------------------------------
# transformers AttentionInterface adapters
# ---------------------------------------------------------------------------
HIP_ATTENTION_NAME = "thundersync_hip"
HIP_FOREST_ATTENTION_NAME = "thundersync_hip_forest"
_PLANS: dict[torch.device, object] = {}


def hip_attention_forward(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Causal attention over one sequence, heads last on the way out.

    The signature and contract of ``fa4_attention_forward``
    (accel/fa4_attention.py:22-53): ``[B, H, T, D]`` in, ``[B, T, H, D]``
    out, grouped K/V heads carried natively, dropout refused.
    """
    if dropout:
        raise ValueError("attention dropout is not supported on this path")
    scale = scaling if scaling is not None else query.shape[-1] ** -0.5
    if query.shape[0] == 1:
        # views whose gradients are views too (an indexed batch row's gradient
        # would be a zero-filled copy of the whole batch)
        o = causal_attention(query, [key.squeeze(0).transpose(0, 1)], [value.squeeze(0).transpose(0, 1)], scale)
        return o.transpose(1, 2), None
    outs = []
    for qb, kb, vb in zip(query.unbind(0), key.unbind(0), value.unbind(0)):
        o = causal_attention(qb.unsqueeze(0), [kb.transpose(0, 1)], [vb.transpose(0, 1)], scale)
        outs.append(o.transpose(1, 2))
    return torch.cat(outs, 0), None


def forest_attention_forward(module, query, key, value, attention_mask, dropout=0.0, scaling=None, **kwargs):
    """HF adapter of engine/step.py:60-99 over the plan bound by :func:`forest_context`."""
    plan = _PLANS.get(query.device)
    if plan is None:
        raise RuntimeError("forest attention was invoked outside `forest_context`")
    if query.shape[0] != 1:
        raise ValueError(f"the forest is already the batch; expected batch dim 1, got {query.shape[0]}")
    out = forest_attention(query.squeeze(0).transpose(0, 1), key.squeeze(0).transpose(0, 1),
                           value.squeeze(0).transpose(0, 1), plan, scale=scaling)
    return out.unsqueeze(0), None


class forest_context:
    """Bind a plan for the duration of a forward (and backward), per device."""

    def __init__(self, plan, device=None):
        self.plan = plan
        self.device = torch.device(device) if device is not None else plan.token_ids.device

    def __enter__(self):
        self.previous = _PLANS.get(self.device)
        _PLANS[self.device] = self.plan
        return self.plan

    def __exit__(self, *exc):
        if self.previous is None:
            _PLANS.pop(self.device, None)
        else:
            _PLANS[self.device] = self.previous
        return False


def register_attention() -> bool:
    """Register both adapters with transformers' AttentionInterface."""
    try:
        from transformers.modeling_utils import AttentionInterface
    except Exception:
        return False
    AttentionInterface.register(HIP_ATTENTION_NAME, hip_attention_forward)
    AttentionInterface.register(HIP_FOREST_ATTENTION_NAME, forest_attention_forward)
    return True
