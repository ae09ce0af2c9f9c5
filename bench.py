#!/usr/bin/env python3
"""Benchmark of the hot path on one MI355X; its last line is ONE JSON summary.

Workloads (synthetic data drawn from fixed seeds):

* ``value``: C2 forest attention, forward + backward -- one shared
  2048-token prompt and 8 sibling completions of lengths U[256, 4096],
  32 query / 8 KV heads, head dim 128, bf16; TFLOP/s counted as
  14 * D * Hq * (exactly visible query/key pairs).
* ``secondary`` rows, by name:
  - ``C4``: chunked retained-KV attention, forward + backward -- 4 groups of
    a 1024-token prompt and 4 completions U[1024, 16384], every 512-token
    query chunk over the group's prompt chunks, its trajectory's earlier
    chunks and itself, K/V held as one tensor per chunk;
  - ``branch_d256``: the reference's own bottom-right branch shape at head
    dim 256 (9288 query rows over 3000 + 9288 keys, 24/4 heads), with
    ``vs_baseline`` against the reference's published FA4 time;
  - ``C3_gated``: fused logprob + entropy, forward + gradient wrt hidden --
    hidden [16384, 4096], head [151936, 4096], 70% of rows scored and gated
    before the projection (the reference's production schedule), frozen
    head; scored tokens/s, 6 * N * V * D FLOP;
  - ``C3_ungated``: the same operator over all 16,384 rows; projected
    tokens/s;
  - ``rmsnorm``: RMSNorm forward + backward on [16384, 4096] bf16; GB/s;
  - ``adjoint``: boundary-adjoint reduction -- an existing parent adjoint
    plus 16 consumer adjoints of [4096, 4096] bf16 summed in fp32 into a new
    tensor; GB/s of inputs read plus output written;
  - ``lora``: merged-weight LoRA linear, forward + backward (dx, dA, dB) at
    a C5 q_proj slice: 16384 tokens, 4096 -> 4096, rank 16;
  - ``C5``: one GRPO-shaped update of the Qwen3-8B-shaped decoder through
    every operator of the build; seconds per update and per-kernel
    breakdown.

Output: one ``bench_detail`` line with every workload's full record
(per-kernel times, configs, device memory), then the summary line the
driver reads, which carries the contract's keys for the headline workload
and one short row per secondary.

The MFMA peak is derived from the device's CU count and peak engine clock
(4096 dense bf16 FLOP per CU per clock), the HBM peak is the published
8 TB/s; both, with their inputs, are in ``peaks``.

A step is one pass of the operator over its whole input, with inputs
already resident in HBM.  Per-kernel device time comes from the library's
own HIP-event brackets (ts_timing_*), recorded on the stream each kernel is
launched on, over the timed steps; ``roofline`` names the kernel with the
largest share.  ``cpu_baseline`` times the CPU oracle (the build's op-for-op
restatement of the reference's eager path) on a bounded sample of the same
workload, on every core the process may run on (``cores``, with
``cpu_model``).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "forest-attn fwd+bwd TFLOP/s; fused-logprob fwd+bwd tokens/s (1 MI355X)"
# Dense bf16 MFMA work per compute unit per engine clock on CDNA4: the
# published 2.5 PFLOP/s of MI355X over its 256 CUs at 2.4 GHz.  The bf16 peak
# is this times the CU count and peak engine clock the device reports.
BF16_FLOP_PER_CU_CLOCK = 4096
PUBLISHED_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0  # published HBM3E bandwidth, MI355X
PEAKS: dict = {}


def device_peaks(device) -> dict:
    """MFMA peak from the device's CU count and engine clock (hipDeviceGetAttribute),
    with the inputs; the HBM peak is the published figure (the reported memory
    clock and bus width are recorded beside it)."""
    from thundersync_amd import _lib

    c = _lib.device_clocks(device.index or 0)
    bf16 = c["cus"] * c["clock_khz"] * 1e3 * BF16_FLOP_PER_CU_CLOCK / 1e12
    return {
        "bf16_tflops": round(bf16, 1),
        "cus": c["cus"],
        "clock_mhz": c["clock_khz"] / 1e3,
        "bf16_flop_per_cu_clock": BF16_FLOP_PER_CU_CLOCK,
        "published_bf16_tflops": PUBLISHED_BF16_TFLOPS,
        "hbm_gbs": PEAK_HBM_GBS,
        "mem_clock_mhz": c["mem_clock_khz"] / 1e3,
        "mem_bus_bits": c["mem_bus_bits"],
    }


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--only", choices=("all", "attention", "chunked", "fa4_branch", "logprob", "logprob_ungated",
                                       "rmsnorm", "adjoint", "lora", "c5", "copy"), default="all",
                    help="one workload; 'copy' runs only the plain 256 MiB device copy whose FETCH_SIZE / "
                         "WRITE_SIZE readings calibrate the traffic counters")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    return ap.parse_args()


def cpu_threads() -> int:
    """Every core this process may run on."""
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:  # pragma: no cover
        pass
    import platform

    return platform.processor() or "unknown"


CPU_BASELINE_SECONDS = 10.0


def repeat_for(fn, seconds=CPU_BASELINE_SECONDS, max_reps=20000):
    """Run `fn` until `seconds` have passed (at least once): (repetitions, elapsed s)."""
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= seconds or reps >= max_reps:
            return reps, dt


def timed(step, steps, warmup, kernels):
    """(ms per step, {kernel: (avg ms per launch, launches per step)}, memory).

    The wall clock times `steps` steps with the library's per-kernel HIP-event
    brackets off (two event records per launch are instrumentation, not the
    job); a second pass of the same steps with the brackets on gives the
    per-kernel device times.  ``memory``: the device memory allocated when
    the timed steps start (inputs, resident state) and the peak allocated
    while they run (``torch.cuda.max_memory_allocated``), in bytes; the
    difference is what a step takes on top (workspaces, activations,
    gradients)."""
    import torch

    from thundersync_amd._lib import KernelTimer

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    resident = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    peak = torch.cuda.max_memory_allocated()
    mem = {"resident_bytes": int(resident), "peak_bytes": int(peak), "step_bytes": int(peak - resident)}
    with KernelTimer():
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        per = {}
        for k in kernels:
            total, n = KernelTimer.read(k)
            if n:
                per[k] = (total / n, n / steps)
    return (t1 - t0) * 1e3 / steps, per, mem


# Sub-millisecond secondaries (RMSNorm, boundary adjoints) repeat their step
# at least this many times, so that the timed region is tens of
# milliseconds rather than a few launch latencies; their JSON records the count.
SHORT_STEPS, SHORT_WARMUP = 200, 20


def measured_entry(workload, kernel) -> dict:
    """The profiles/traffic.json entry of `kernel` in `workload` ({} when none):
    HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs
    of this script with ``--only <workload>``, each scaled by what the counter
    reads for a plain device copy of known size, and, where measured, the
    engine clock the kernel ran at (GRBM_GUI_ACTIVE cycles per XCD over the
    dispatch's duration)."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return {}
    table = json.loads(path.read_text())
    return table.get("workloads", {}).get(workload, {}).get(kernel) or {}


def roofline_of(per, work_per_step, unit, peak, workload):
    """Roofline object for the kernel with the largest device time per step.

    ``work_per_step`` is the kernel's algorithmic work over one step; a kernel
    launched several times per step (the logprob backward runs one launch per
    row block) does that work split over its launches.
    """
    name = max(per, key=lambda k: per[k][0] * per[k][1])
    avg_ms, launches = per[name]
    per_launch = work_per_step[name] / launches
    achieved = per_launch / (avg_ms * 1e-3) / (1e12 if unit == "TFLOP/s" else 1e9)
    entry = measured_entry(workload, name)
    traffic = entry.get("traffic_bytes")
    out = {
        "kernel": name,
        "bound": "mfma" if unit == "TFLOP/s" else "hbm",
        "achieved": round(achieved, 2),
        "peak": peak,
        "unit": unit,
        "frac": round(achieved / peak, 4),
        "traffic": traffic,
        "traffic_source": (f"profiles/traffic.json, measured at commit {entry.get('measured_at_commit')}"
                           if traffic is not None else None),
        "avg_launch_ms": round(avg_ms, 4),
        "launches_per_step": launches,
        "work_per_launch": per_launch,
    }
    clock = entry.get("clock_mhz")
    if clock and unit == "TFLOP/s":
        # context, not the roofline: the MFMA peak at the clock the chip held
        # while this kernel ran, and the kernel's fraction of that
        out["sustained_clock_mhz"] = round(clock)
        out["frac_at_sustained_clock"] = round(achieved / (peak * clock / PEAKS["clock_mhz"]), 4)
    return out


# ---------------------------------------------------------------------------
# C2 forest attention
# ---------------------------------------------------------------------------
def c2_inputs(seed, device):
    import torch

    from thundersync_amd import forest

    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(256, 4097, (8,), generator=g).tolist()
    prompt = torch.randint(0, 100000, (2048,), generator=g).tolist()
    trajs = []
    for i, n in enumerate(lengths):
        body = [100000 + i] + torch.randint(0, 100000, (n - 1,), generator=g).tolist()
        trajs.append(forest.Trajectory([forest.Segment.prompt(prompt), forest.Segment.action(body)],
                                       group_id=0, traj_id=i))
    plan = forest.compile_plan(forest.build_forest(trajs))
    p = plan.n_physical
    gd = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(p, 32, 128, generator=gd, device=device, dtype=torch.bfloat16).requires_grad_()
    k = torch.randn(p, 8, 128, generator=gd, device=device, dtype=torch.bfloat16).requires_grad_()
    v = torch.randn(p, 8, 128, generator=gd, device=device, dtype=torch.bfloat16).requires_grad_()
    dout = torch.randn(p, 32, 128, generator=gd, device=device, dtype=torch.bfloat16)
    return plan, lengths, q, k, v, dout


def bench_attention(args, device):
    import torch

    from thundersync_amd import attention

    plan, lengths, q, k, v, dout = c2_inputs(args.seed, device)
    layout = attention.forest_layout(plan, 32, 8)
    pairs = layout.visible_pairs()
    d, hq = 128, 32

    def step():
        q.grad = k.grad = v.grad = None
        out = attention.forest_attention(q, k, v, plan)
        out.backward(dout)

    kernels = ["attention.fwd_kernel", "attention.delta_kernel", "attention.dq_kernel", "attention.dkdv_kernel"]
    ms, per, mem = timed(step, args.steps, args.warmup, kernels)
    flop = 14 * d * hq * pairs
    work = {
        "attention.fwd_kernel": 4 * d * hq * pairs,
        "attention.dq_kernel": 2 * d * hq * pairs,
        "attention.dkdv_kernel": 8 * d * hq * pairs,
        "attention.delta_kernel": 2 * d * hq * plan.n_physical,
    }
    result = {
        "value": round(flop / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "memory": mem,
        "roofline": roofline_of(per, work, "TFLOP/s", PEAKS["bf16_tflops"], "attention"),
        "kernels": {k: {"avg_ms": round(a, 4), "launches_per_step": n} for k, (a, n) in per.items()},
        "config": {
            "workload": "C2 forest attention fwd+bwd: 2048-token shared prompt + 8 completions "
                        "U[256,4096], 32/8 heads, head_dim 128, bf16",
            "completion_lengths": lengths,
            "tokens": plan.n_physical,
            "visible_pairs": pairs,
            "flop_per_step": flop,
            "seed": args.seed,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = attention_cpu_baseline(plan, q, k, v, dout, lengths)
    return result


def attention_cpu_baseline(plan, q, k, v, dout, lengths):
    """The reference's CPU dispatch (masked SDPA, causal_lower_right, GQA by
    repeat_interleave; engine/streaming.py:1146-1162) on the prompt node and
    the first completion node, fp32, forward + backward."""
    import torch

    from oracle import attention as ref

    torch.set_num_threads(cpu_threads())
    qc, kc, vc, dc = (t.detach().float().cpu() for t in (q, k, v, dout))
    starts, ends = plan.node_start.tolist(), plan.node_end.tolist()
    work = []
    for n in (0, 1):
        s, e = starts[n], ends[n]
        keys = [(a, b) for a, b in plan.key_ranges[n] if b > a]
        work.append((s, e, keys))
    pairs = sum((e - s) * (sum(b - a for a, b in keys) - (e - s)) + (e - s) * (e - s + 1) // 2
                for s, e, keys in work)
    def one_pass():
        for s, e, keys in work:
            qq = qc[s:e].clone().requires_grad_()
            kk = torch.cat([kc[a:b] for a, b in keys]).requires_grad_()
            vv = torch.cat([vc[a:b] for a, b in keys]).requires_grad_()
            out = ref.sdpa_lower_right(qq, kk, vv, 128 ** -0.5)
            torch.autograd.grad(out, (qq, kk, vv), dc[s:e])

    reps, dt = repeat_for(one_pass)
    return {
        "value": round(14 * 128 * 32 * pairs * reps / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"prompt node (2048 rows) + first completion node ({lengths[0]} rows) of the same C2 "
                  f"forest, {pairs} visible pairs, fp32 masked SDPA fwd+bwd on the host, {reps} passes",
        "seconds": round(dt, 3),
    }


# ---------------------------------------------------------------------------
# the reference's bottom-right branch shape (its FA4 headline figure)
# ---------------------------------------------------------------------------
FA4_BRANCH = {"prefix": 3000, "tail": 9288, "hq": 24, "hkv": 4, "head_dim": 256}
# the reference's published fwd+bwd time at this shape, FA4 on unstated NVIDIA
# hardware (tests/test_fa4_bottom_right.py:50-55 of the reference)
FA4_BRANCH_REFERENCE_MS = 7.023


def bench_fa4_branch(args, device):
    """A query tail over prefix + tail keys, bottom-right causal, 24/4 heads,
    head dim 256, bf16 (tests/test_fa4_bottom_right.py:13-28 of the reference),
    forward + backward through the callable-backend form ``causal_attention``."""
    import torch

    from thundersync_amd import attention

    c = FA4_BRANCH
    prefix, tail, hq, hkv, d = c["prefix"], c["tail"], c["hq"], c["hkv"], c["head_dim"]
    g = torch.Generator(device=device).manual_seed(args.seed)
    q = torch.randn(1, hq, tail, d, device=device, dtype=torch.bfloat16, generator=g).requires_grad_()
    k = torch.randn(prefix + tail, hkv, d, device=device, dtype=torch.bfloat16, generator=g).requires_grad_()
    v = torch.randn(prefix + tail, hkv, d, device=device, dtype=torch.bfloat16, generator=g).requires_grad_()
    dout = torch.randn(1, hq, tail, d, device=device, dtype=torch.bfloat16, generator=g)
    scale = d ** -0.5
    pairs = tail * prefix + tail * (tail + 1) // 2

    def step():
        q.grad = k.grad = v.grad = None
        out = attention.causal_attention(q, [k], [v], scale)
        out.backward(dout)

    kernels = ["attention.fwd_kernel", "attention.delta_kernel", "attention.dq_kernel", "attention.dkdv_kernel"]
    ms, per, mem = timed(step, args.steps, args.warmup, kernels)
    flop = 14 * d * hq * pairs
    work = {
        "attention.fwd_kernel": 4 * d * hq * pairs,
        "attention.dq_kernel": 2 * d * hq * pairs,
        "attention.dkdv_kernel": 8 * d * hq * pairs,
        "attention.delta_kernel": 2 * d * hq * tail,
    }
    tflops = flop / (ms * 1e-3) / 1e12
    reference_tflops = flop / (FA4_BRANCH_REFERENCE_MS * 1e-3) / 1e12
    result = {
        "metric": "bottom-right branch attention fwd+bwd TFLOP/s (the reference's FA4 shape)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "memory": mem,
        "vs_baseline": round(tflops / reference_tflops, 4),
        "baseline": {"ms": FA4_BRANCH_REFERENCE_MS, "tflops": round(reference_tflops, 1),
                     "what": "the reference's FA4 fwd+bwd at this shape on unstated NVIDIA hardware "
                             "(tests/test_fa4_bottom_right.py:50-55)"},
        "roofline": roofline_of(per, work, "TFLOP/s", PEAKS["bf16_tflops"], "fa4_branch"),
        "kernels": {k: {"avg_ms": round(a, 4), "launches_per_step": n} for k, (a, n) in per.items()},
        "config": {
            "workload": f"bottom-right branch attention fwd+bwd: {tail} query rows over {prefix} prefix + {tail} "
                        f"keys, {hq}/{hkv} heads, head_dim {d}, bf16",
            "visible_pairs": pairs,
            "flop_per_step": flop,
            "seed": args.seed,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = fa4_branch_cpu_baseline(q, k, v, dout, scale, prefix)
    return result


def fa4_branch_cpu_baseline(q, k, v, dout, scale, prefix, rows=192):
    """The reference's CPU dispatch (masked SDPA, causal_lower_right, GQA by
    repeat_interleave; engine/streaming.py:1146-1162) on the first ``rows``
    query rows of the tail over the keys they see, fp32, forward + backward."""
    import torch

    from oracle import attention as ref

    torch.set_num_threads(cpu_threads())
    hq, d = q.shape[1], q.shape[3]
    qq0 = q[0, :, :rows].detach().transpose(0, 1).float().cpu().contiguous()
    kk0 = k[: prefix + rows].detach().float().cpu()
    vv0 = v[: prefix + rows].detach().float().cpu()
    dd = dout[0, :, :rows].detach().transpose(0, 1).float().cpu().contiguous()
    pairs = rows * prefix + rows * (rows + 1) // 2

    def one_pass():
        qq, kk, vv = (t.clone().requires_grad_() for t in (qq0, kk0, vv0))
        out = ref.sdpa_lower_right(qq, kk, vv, scale)
        torch.autograd.grad(out, (qq, kk, vv), dd)

    reps, dt = repeat_for(one_pass)
    return {
        "value": round(14 * d * hq * pairs * reps / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"the first {rows} query rows of the tail over their {prefix} + {rows} keys ({pairs} visible "
                  f"pairs), fp32 masked SDPA fwd+bwd on the host, {reps} passes",
        "seconds": round(dt, 3),
    }


# ---------------------------------------------------------------------------
# C4 chunked retained-KV attention
# ---------------------------------------------------------------------------
def c4_layout(seed, chunk=512, groups=4, per_group=4, prompt=1024, lo=1024, hi=16384):
    """(lengths, chunk_rows, query chunks, q_rows) of the C4 pack.

    Each group's prompt and each trajectory is cut into `chunk`-token query
    chunks; a chunk reads the group's prompt chunks, the earlier chunks of
    its trajectory and itself (bottom-right causal).  Rows are laid out group
    by group: prompt, then its trajectories in order.
    """
    import torch

    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(lo, hi + 1, (groups * per_group,), generator=g).tolist()
    chunk_rows, chunks, row = [], [], 0

    def cut(n, path):
        nonlocal row
        for c0 in range(0, n, chunk):
            m = min(chunk, n - c0)
            chunk_rows.append(m)
            path.append(len(chunk_rows) - 1)
            chunks.append((row, m, tuple(path)))
            row += m

    for grp in range(groups):
        prompt_path = []
        cut(prompt, prompt_path)
        for t in range(per_group):
            cut(lengths[grp * per_group + t], list(prompt_path))
    return lengths, chunk_rows, chunks, row


def c4_inputs(seed, device):
    import torch

    from thundersync_amd import attention

    lengths, chunk_rows, chunks, rows = c4_layout(seed)
    layout = attention.retained_chunk_layout(rows, chunk_rows, chunks, 32, 8)
    gd = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(rows, 32, 128, generator=gd, device=device, dtype=torch.bfloat16).requires_grad_()
    ks = [torch.randn(n, 8, 128, generator=gd, device=device, dtype=torch.bfloat16).requires_grad_()
          for n in chunk_rows]
    vs = [torch.randn(n, 8, 128, generator=gd, device=device, dtype=torch.bfloat16).requires_grad_()
          for n in chunk_rows]
    dout = torch.randn(rows, 32, 128, generator=gd, device=device, dtype=torch.bfloat16)
    return lengths, chunks, layout, q, ks, vs, dout


def bench_chunked(args, device):
    import torch

    from thundersync_amd import attention

    lengths, chunks, layout, q, ks, vs, dout = c4_inputs(args.seed, device)
    pairs = layout.visible_pairs()
    d, hq = 128, 32
    leaves = [q, *ks, *vs]

    def step():
        for t in leaves:
            t.grad = None
        out = attention.retained_chunk_attention(q, ks, vs, layout, 128 ** -0.5)
        out.backward(dout)

    kernels = ["attention.fwd_kernel", "attention.delta_kernel", "attention.dq_kernel", "attention.dkdv_kernel"]
    ms, per, mem = timed(step, args.steps, args.warmup, kernels)
    flop = 14 * d * hq * pairs
    work = {
        "attention.fwd_kernel": 4 * d * hq * pairs,
        "attention.dq_kernel": 2 * d * hq * pairs,
        "attention.dkdv_kernel": 8 * d * hq * pairs,
        "attention.delta_kernel": 2 * d * hq * layout.q_rows,
    }
    result = {
        "metric": "chunked retained-KV attn fwd+bwd TFLOP/s",
        "value": round(flop / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "memory": mem,
        "roofline": roofline_of(per, work, "TFLOP/s", PEAKS["bf16_tflops"], "chunked"),
        "kernels": {k: {"avg_ms": round(a, 4), "launches_per_step": n} for k, (a, n) in per.items()},
        "config": {
            "workload": "C4 chunked retained-KV attention fwd+bwd: 4 groups x (1024-token prompt + 4 "
                        "completions U[1024,16384]), 512-token query chunks over per-chunk K/V tensors, "
                        "32/8 heads, head_dim 128, bf16, all chunks in one launch per direction",
            "completion_lengths": lengths,
            "tokens": layout.q_rows,
            "query_chunks": len(chunks),
            "visible_pairs": pairs,
            "flop_per_step": flop,
            "seed": args.seed,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = chunked_cpu_baseline(chunks, lengths, q, ks, vs, dout)
    return result


def chunked_cpu_baseline(chunks, lengths, q, ks, vs, dout, chunk=512, prompt=1024):
    """The reference's CPU dispatch (masked SDPA, causal_lower_right;
    engine/streaming.py:1146-1162) on every query chunk of the first
    trajectory, each over the concatenation of its retained K/V, fp32
    forward + backward."""
    import torch

    from oracle import attention as ref

    torch.set_num_threads(cpu_threads())
    # group 0 lays out its prompt chunks first, then the first trajectory's chunks
    first = prompt // chunk
    last = first + -(-lengths[0] // chunk)
    sample = list(range(first, last))
    host, pairs = [], 0
    for i in sample:
        row0, m, path = chunks[i]
        qq = q.detach()[row0 : row0 + m].float().cpu()
        kk = [ks[c].detach().float().cpu() for c in path]
        vv = [vs[c].detach().float().cpu() for c in path]
        s = sum(k.shape[0] for k in kk)
        pairs += m * (s - m) + m * (m + 1) // 2
        host.append((qq, kk, vv, dout[row0 : row0 + m].float().cpu()))
    def one_pass():
        for qq, kk, vv, dd in host:
            qq = qq.detach().requires_grad_()
            kc = torch.cat(kk).requires_grad_()  # the reference's ancestor cat
            vc = torch.cat(vv).requires_grad_()
            out = ref.sdpa_lower_right(qq, kc, vc, 128 ** -0.5)
            torch.autograd.grad(out, (qq, kc, vc), dd)

    reps, dt = repeat_for(one_pass)
    return {
        "value": round(14 * 128 * 32 * pairs * reps / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"the {len(sample)} query chunks of the first C4 trajectory ({pairs} visible pairs), "
                  f"fp32 masked SDPA fwd+bwd over the concatenated retained K/V on the host, {reps} passes",
        "seconds": round(dt, 3),
    }


# ---------------------------------------------------------------------------
# C3 fused logprob
# ---------------------------------------------------------------------------
def bench_logprob(args, device, gate: bool = True):
    """C3: ``gate`` projects only the scored rows (70%), the reference's
    production schedule; ``gate=False`` projects all 16,384 rows, the
    ungated form."""
    import torch

    from thundersync_amd import fused_logprob

    n, d, v = 16384, 4096, 151936
    g = torch.Generator(device=device).manual_seed(args.seed)
    hidden = torch.randn(n, d, generator=g, device=device, dtype=torch.bfloat16)
    weight = (torch.randn(v, d, generator=g, device=device) * 0.02).to(torch.bfloat16)
    target = torch.randint(0, v, (n,), generator=g, device=device)
    adv = torch.randn(n, generator=g, device=device)
    mask = torch.rand(n, generator=g, device=device) < 0.7
    idx = mask.nonzero(as_tuple=True)[0] if gate else torch.arange(n, device=device)
    h = hidden.index_select(0, idx).requires_grad_()
    t = target.index_select(0, idx)
    a = adv.index_select(0, idx)
    rows = int(idx.numel())

    def step():
        h.grad = None
        lp, ent = fused_logprob.fused_logprob_entropy(h, weight, t)
        lp.backward(a)

    kernels = ["logprob.fwd_stats_kernel", "logprob.target_logit_kernel", "logprob.combine_kernel",
               "logprob.dlogits_kernel", "logprob.grad_hidden_kernel", "logprob.grad_hidden_reduce_kernel"]
    ms, per, mem = timed(step, args.steps, args.warmup, kernels)
    gemm = 2 * rows * v * d
    work = {
        "logprob.fwd_stats_kernel": gemm,
        "logprob.dlogits_kernel": gemm,
        "logprob.grad_hidden_kernel": gemm,
        "logprob.combine_kernel": 0,
        "logprob.target_logit_kernel": 0,
        "logprob.grad_hidden_reduce_kernel": 0,
    }
    flop = 3 * gemm
    form = ("70% scored rows gated first" if gate else "all 16384 rows projected (ungated)")
    result = {
        "metric": "fused-logprob fwd+bwd tokens/s" + ("" if gate else " (ungated)"),
        "value": round(rows / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
        "mfma_frac": round(flop / (ms * 1e-3) / 1e12 / PEAKS["bf16_tflops"], 4),
        "ms_per_step": round(ms, 4),
        "memory": mem,
        "roofline": roofline_of({k: x for k, x in per.items() if work[k]}, work, "TFLOP/s", PEAKS["bf16_tflops"],
                                "logprob" if gate else "logprob_ungated"),
        "kernels": {k: {"avg_ms": round(x, 4), "launches_per_step": m} for k, (x, m) in per.items()},
        "config": {
            "workload": "C3 fused logprob+entropy fwd + grad wrt hidden: hidden [16384,4096] bf16, "
                        f"head [151936,4096] bf16 N(0,0.02), {form}, frozen head",
            "projected_rows": rows,
            "flop_per_step": flop,
            "seed": args.seed,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = logprob_cpu_baseline(h, weight, t, a)
    return result


def logprob_cpu_baseline(h, weight, t, a, rows=96):
    """The reference's chunk loop (accel/fused_logprob.py:250-308, CPU branch)
    on the first `rows` scored rows, fwd + backward wrt hidden."""
    import torch

    from oracle import logprob as ref

    torch.set_num_threads(cpu_threads())
    hs = h.detach()[:rows].cpu()
    w = weight.cpu()
    ts = t[:rows].cpu()
    g = a[:rows].cpu()
    def one_pass():
        lp, ent = ref.logprob_entropy_forward(hs, w, ts, 1024)
        ref.logprob_entropy_backward(hs, w, ts, ent, g, torch.zeros(rows), 1024)

    reps, dt = repeat_for(one_pass)
    return {
        "value": round(rows * reps / dt, 2),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"{rows} scored rows of C3 (dim 4096, vocab 151936), chunk 1024, fwd + grad wrt hidden, "
                  f"{reps} passes",
        "seconds": round(dt, 3),
    }


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
def bench_rmsnorm(args, device):
    import torch

    from thundersync_amd import rms_norm

    r, w_ = 16384, 4096
    g = torch.Generator(device=device).manual_seed(args.seed)
    x = torch.randn(r, w_, generator=g, device=device, dtype=torch.bfloat16).requires_grad_()
    w = torch.linspace(0.4, 3.0, w_, device=device).to(torch.bfloat16).requires_grad_()
    dy = torch.randn(r, w_, generator=g, device=device, dtype=torch.bfloat16)

    def step():
        x.grad = w.grad = None
        y = rms_norm.FP32RMSNormVJP.apply(x, w, 1e-6)
        y.backward(dy)

    kernels = ["rmsnorm.rmsnorm_fwd_lanes", "rmsnorm.rmsnorm_fwd_rowwave", "rmsnorm.rmsnorm_bwd_vec",
               "rmsnorm.rmsnorm_dw_reduce"]
    steps, warmup = max(args.steps, SHORT_STEPS), max(args.warmup, SHORT_WARMUP)
    ms, per, mem = timed(step, steps, warmup, kernels)
    fwd_bytes = 4 * r * w_ + 4 * r + 2 * w_
    bwd_bytes = 6 * r * w_ + 4 * r + 2 * w_ + 4 * w_
    work = {"rmsnorm.rmsnorm_fwd_lanes": fwd_bytes, "rmsnorm.rmsnorm_fwd_rowwave": fwd_bytes,
            "rmsnorm.rmsnorm_bwd_vec": bwd_bytes, "rmsnorm.rmsnorm_dw_reduce": 0}
    result = {
        "metric": "RMSNorm fwd+bwd GB/s",
        "value": round((fwd_bytes + bwd_bytes) / (ms * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "ms_per_step": round(ms, 4),
        "memory": mem,
        "roofline": roofline_of({k: x for k, x in per.items() if work[k]}, work, "GB/s", PEAKS["hbm_gbs"], "rmsnorm"),
        "kernels": {k: {"avg_ms": round(x, 4), "launches_per_step": m} for k, (x, m) in per.items()},
        "steps": steps,
        "warmup": warmup,
        "config": {"workload": "RMSNorm fwd+bwd [16384, 4096] bf16, FP32 VJP with dW", "seed": args.seed},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = rmsnorm_cpu_baseline(x, w, dy, (fwd_bytes + bwd_bytes) / r)
    return result


def rmsnorm_cpu_baseline(x, w, dy, bytes_per_row, rows=2048):
    """The reference's eager forward (accel/rms_norm.py:11-14) and FP32 VJP
    (:33-38) on the CPU over the first `rows` rows; GB/s of the same
    algorithmic bytes per row as the device figure."""
    import torch

    from oracle import rms_norm as ref

    torch.set_num_threads(cpu_threads())
    xs, ws, gs = x.detach()[:rows].cpu(), w.detach().cpu(), dy[:rows].cpu()

    def one_pass():
        ref.rms_norm_forward(xs, ws, 1e-6)
        ref.rms_norm_backward(gs, xs, ws, 1e-6)

    reps, dt = repeat_for(one_pass)
    return {
        "value": round(bytes_per_row * rows * reps / dt / 1e9, 2),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"first {rows} of 16384 rows of [16384, 4096] bf16, eager fp32 forward + VJP, {reps} passes",
        "seconds": round(dt, 3),
    }


# ---------------------------------------------------------------------------
# Boundary-adjoint reduction
# ---------------------------------------------------------------------------
ADJOINT_DEGREE = 16
ADJOINT_SHAPE = (4096, 4096)


def bench_adjoint(args, device):
    import torch

    from thundersync_amd import boundary_adjoint

    g = torch.Generator(device=device).manual_seed(args.seed)
    adj = [torch.randn(ADJOINT_SHAPE, generator=g, device=device, dtype=torch.bfloat16)
           for _ in range(ADJOINT_DEGREE)]
    existing = torch.randn(ADJOINT_SHAPE, generator=g, device=device, dtype=torch.bfloat16)

    def step():
        boundary_adjoint.reduce_boundary_adjoints(adj, existing=existing)

    kernels = ["adjoint.reduce_kernel"]
    steps, warmup = max(args.steps, SHORT_STEPS), max(args.warmup, SHORT_WARMUP)
    ms, per, mem = timed(step, steps, warmup, kernels)
    n = ADJOINT_SHAPE[0] * ADJOINT_SHAPE[1]
    nbytes = (ADJOINT_DEGREE + 1) * n * 2 + n * 2  # every input read once, the output written once
    result = {
        "metric": "boundary-adjoint reduce GB/s",
        "value": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "ms_per_step": round(ms, 4),
        "memory": mem,
        "roofline": roofline_of(per, {"adjoint.reduce_kernel": nbytes}, "GB/s", PEAKS["hbm_gbs"], "adjoint"),
        "kernels": {k: {"avg_ms": round(x, 4), "launches_per_step": m} for k, (x, m) in per.items()},
        "steps": steps,
        "warmup": warmup,
        "config": {"workload": f"boundary adjoint: existing + {ADJOINT_DEGREE} consumer adjoints "
                               f"[{ADJOINT_SHAPE[0]}, {ADJOINT_SHAPE[1]}] bf16, fp32 accumulation",
                   "seed": args.seed},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = adjoint_cpu_baseline(adj, existing, nbytes)
    return result


def adjoint_cpu_baseline(adj, existing, nbytes, rows=1024):
    """The fused reduction's semantics on the CPU (engine/boundary_adjoint.py:75-115:
    fp32 accumulation in input order, one cast) over the first `rows` rows."""
    import torch

    from oracle import boundary_adjoint as ref

    torch.set_num_threads(cpu_threads())
    a = [x[:rows].cpu() for x in adj]
    e = existing[:rows].cpu()
    reps, dt = repeat_for(lambda: ref.reduce_fp32(a, e))
    sample_bytes = nbytes * rows / ADJOINT_SHAPE[0]
    return {
        "value": round(sample_bytes * reps / dt / 1e9, 2),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"first {rows} of {ADJOINT_SHAPE[0]} rows, existing + {ADJOINT_DEGREE} bf16 adjoints, "
                  f"{reps} passes",
        "seconds": round(dt, 3),
    }


# ---------------------------------------------------------------------------
# Merged-weight LoRA linear
# ---------------------------------------------------------------------------
LORA_SHAPE = (16384, 4096, 4096, 16)  # tokens, in, out, rank: a C5 q_proj over 16384 tokens


def bench_lora(args, device):
    import torch

    from thundersync_amd import fused_lora

    t, fin, fout, r = LORA_SHAPE
    g = torch.Generator(device=device).manual_seed(args.seed)
    x = torch.randn(t, fin, generator=g, device=device, dtype=torch.bfloat16).requires_grad_()
    w = (torch.randn(fout, fin, generator=g, device=device) * fin ** -0.5).to(torch.bfloat16)
    a = (torch.randn(r, fin, generator=g, device=device) * fin ** -0.5).requires_grad_()
    b = (torch.randn(fout, r, generator=g, device=device) * 0.01).requires_grad_()
    dy = torch.randn(t, fout, generator=g, device=device, dtype=torch.bfloat16)

    def step():
        x.grad = a.grad = b.grad = None
        fused_lora.FusedLoRALinear.apply(x, w, a, b, 2.0).backward(dy)

    kernels = ["lora.fwd_kernel", "lora.grad_x_kernel", "lora.grad_x_reduce_kernel", "lora.rank_kernel",
               "lora.grad_a_kernel", "lora.grad_b_kernel", "lora.reduce_kernel"]
    ms, per, mem = timed(step, args.steps, args.warmup, kernels)
    gemm = 2 * t * fin * fout
    adapter = 2 * t * r * (fin + fout)  # g B and x A^T, then u^T x and g^T t: the same count again
    work = {"lora.fwd_kernel": gemm, "lora.grad_x_kernel": gemm, "lora.rank_kernel": adapter,
            "lora.grad_a_kernel": 2 * t * r * fin, "lora.grad_b_kernel": 2 * t * r * fout,
            "lora.grad_x_reduce_kernel": 0, "lora.reduce_kernel": 0}
    flop = 2 * gemm + 2 * adapter
    # the adapter products read g and x (bf16) twice over the backward
    adapter_bytes = 2 * 2 * t * (fin + fout)
    adapter_ms = sum(per[k][0] * per[k][1] for k in ("lora.rank_kernel", "lora.grad_a_kernel",
                                                      "lora.grad_b_kernel", "lora.reduce_kernel") if k in per)
    result = {
        "metric": "merged-weight LoRA linear fwd+bwd TFLOP/s",
        "value": round(flop / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOP/s",
        "ms_per_step": round(ms, 4),
        "memory": mem,
        "roofline": roofline_of({k: v for k, v in per.items() if work[k]}, work, "TFLOP/s", PEAKS["bf16_tflops"],
                                "lora"),
        "adapter_gradients": {"ms": round(adapter_ms, 4), "bytes": adapter_bytes,
                              "gbs": round(adapter_bytes / (adapter_ms * 1e-3) / 1e9, 1) if adapter_ms else None},
        "kernels": {k: {"avg_ms": round(v, 4), "launches_per_step": n} for k, (v, n) in per.items()},
        "config": {"workload": f"FusedLoRALinear fwd + bwd (dx, dA, dB): x [{t}, {fin}] bf16, W_eff [{fout}, {fin}] "
                               f"bf16, rank {r} fp32 adapters, scaling 2 (a C5 q_proj slice)",
                   "flop_per_step": flop, "seed": args.seed},
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = lora_cpu_baseline(x, w, a, b, dy, flop / t)
    return result


def lora_cpu_baseline(x, w, a, b, dy, flop_per_row, rows=512):
    """The reference layer's forward + backward (accel/fused_lora.py:29-48) on
    the CPU in fp32 over the first `rows` rows."""
    import torch

    from oracle import lora as ref

    torch.set_num_threads(cpu_threads())
    xs, ws, gs = x.detach()[:rows].float().cpu(), w.float().cpu(), dy[:rows].float().cpu()
    as_, bs = a.detach().cpu(), b.detach().cpu()
    reps, dt = repeat_for(lambda: ref.reference_step(xs, ws, as_, bs, gs, 2.0))
    return {
        "value": round(flop_per_row * rows * reps / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": f"first {rows} of {LORA_SHAPE[0]} rows, fp32 eager forward + backward, {reps} passes",
        "seconds": round(dt, 3),
    }


# ---------------------------------------------------------------------------
# C5: one GRPO-shaped update of a Qwen3-8B-shaped decoder (opt-in: --only c5)
# ---------------------------------------------------------------------------
def c5_model(device):
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from thundersync_amd.attention import HIP_FOREST_ATTENTION_NAME, register_attention
    from thundersync_amd.lora_layers import add_lora
    from thundersync_amd.rms_norm import use_stable_qwen3_rms_norm

    cfg = Qwen3Config(vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=36,
                      num_attention_heads=32, num_key_value_heads=8, head_dim=128, tie_word_embeddings=False,
                      max_position_embeddings=40960, rms_norm_eps=1e-6)
    default = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen3ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(default)
    assert register_attention()
    model.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)
    use_stable_qwen3_rms_norm(model)
    add_lora(model, ["q_proj", "k_proj", "v_proj", "o_proj"], rank=16, alpha=32)
    model.gradient_checkpointing_enable(gradient_checkpointing_kwargs={"use_reentrant": False})
    model.train()
    return model


def c5_rollouts(seed, device):
    import torch

    from thundersync_amd import forest

    g = torch.Generator().manual_seed(seed)
    trajs, rewards = [], []
    for grp in range(2):
        prompt = torch.randint(0, 151936, (1024,), generator=g).tolist()
        lengths = torch.randint(512, 8193, (8,), generator=g).tolist()
        for i, n in enumerate(lengths):
            body = torch.randint(0, 151936, (n,), generator=g).tolist()
            trajs.append(forest.Trajectory([forest.Segment.prompt(prompt), forest.Segment.action(body)],
                                           group_id=grp, traj_id=8 * grp + i))
        rewards.append(torch.randn(8, generator=g))
    r = torch.stack(rewards)
    adv = ((r - r.mean(1, keepdim=True)) / r.std(1, unbiased=False, keepdim=True).clamp_min(1e-6)).flatten()
    plan = forest.compile_plan(forest.build_forest(trajs)).to(device)
    return plan, {i: float(adv[i]) for i in range(16)}


def bench_c5(args, device):
    import torch

    from thundersync_amd import attention as att
    from thundersync_amd.attention import forest_context
    from thundersync_amd.fused_lora import fuse_merged_lora_forward, unfuse_merged_lora_forward
    from thundersync_amd.step import forest_logprobs, split_by_trajectory

    t0 = time.perf_counter()
    model = c5_model(device)
    plan, adv = c5_rollouts(args.seed, device)
    build_s = time.perf_counter() - t0
    params = [p for p in model.parameters() if p.requires_grad]
    opt = torch.optim.AdamW(params, lr=1e-5)
    scored = int(plan.score_src.numel())

    def update():
        fuse_merged_lora_forward(model)
        with forest_context(plan):
            lp = forest_logprobs(model, plan)
            per = split_by_trajectory(plan, lp)
            loss = -sum(adv[tid] * v.sum() for tid, v in per.items()) / lp.numel()
            loss.backward()
        unfuse_merged_lora_forward(model)
        opt.step()
        opt.zero_grad(set_to_none=True)

    kernels = ["attention.fwd_kernel", "attention.delta_kernel", "attention.dq_kernel", "attention.dkdv_kernel",
               "logprob.fwd_stats_kernel", "logprob.target_logit_kernel", "logprob.combine_kernel",
               "logprob.dlogits_kernel", "logprob.grad_hidden_kernel", "logprob.grad_hidden_reduce_kernel",
               "rmsnorm.rmsnorm_fwd_lanes", "rmsnorm.rmsnorm_fwd_rowwave", "rmsnorm.rmsnorm_bwd_vec",
               "rmsnorm.rmsnorm_bwd_scalar", "rmsnorm.rmsnorm_dw_reduce",
               "lora.fwd_kernel", "lora.grad_x_kernel", "lora.grad_x_reduce_kernel", "lora.rank_kernel",
               "lora.grad_a_kernel", "lora.grad_b_kernel", "lora.reduce_kernel"]
    steps, warmup = max(1, min(args.steps, 3)), max(1, min(args.warmup, 1))
    ms, per, mem = timed(update, steps, warmup, kernels)
    p, layers, d, hq = plan.n_physical, 36, 128, 32
    pairs = att.forest_layout(plan, 32, 8).visible_pairs()
    proj = 2 * p * (4096 * 4096 * 2 + 4096 * 1024 * 2)  # q, k, v, o of one layer
    v, dim = 151936, 4096
    work = {  # per update; the forward of every layer runs twice (checkpoint recompute)
        "attention.fwd_kernel": 2 * layers * 4 * d * hq * pairs,
        "attention.dq_kernel": layers * 2 * d * hq * pairs,
        "attention.dkdv_kernel": layers * 8 * d * hq * pairs,
        "lora.fwd_kernel": 2 * layers * proj,
        "lora.grad_x_kernel": layers * proj,
        "logprob.fwd_stats_kernel": 2 * scored * v * dim,
        "logprob.dlogits_kernel": 2 * scored * v * dim,
        "logprob.grad_hidden_kernel": 2 * scored * v * dim,
    }
    kern = {}
    for k, (avg, n) in per.items():
        entry = {"avg_ms": round(avg, 4), "launches_per_update": n, "ms_per_update": round(avg * n, 3)}
        if k in work:
            tf = work[k] / (avg * n * 1e-3) / 1e12
            entry.update(tflops=round(tf, 1), frac=round(tf / PEAKS["bf16_tflops"], 4))
        kern[k] = entry
    ours = sum(e["ms_per_update"] for e in kern.values())
    model_flop = 6 * 6.95e9 * p  # dense linears fwd + recompute + dx, order of magnitude only
    return {
        "metric": "C5 GRPO update wall time (one MI355X)",
        "value": round(ms / 1e3, 3),
        "unit": "s",
        "higher_is_better": False,
        "ms_per_step": round(ms, 1),
        "memory": mem,
        "library_kernel_ms": round(ours, 1),
        "other_ms": round(ms - ours, 1),
        "kernels": kern,
        "config": {"workload": "Qwen3-8B-shaped decoder (36 layers, 4096, 32/8 heads, MLP 12288, vocab 151936), "
                               "random-init bf16, LoRA rank 16 on q/k/v/o (fp32 adapters, merged-weight path), "
                               "2 groups x 8 trajectories, prompt 1024, completions U[512,8192], forest attention, "
                               "fused logprob, HIP RMSNorm, per-layer activation checkpointing, AdamW on the adapters",
                   "physical_tokens": p, "logical_tokens": plan.forest.logical_tokens, "scored_tokens": scored,
                   "visible_pairs_per_layer": pairs, "build_seconds": round(build_s, 1),
                   "steps": steps, "warmup": warmup, "seed": args.seed,
                   "approx_dense_linear_flop": model_flop},
    }


def calibration_copy(device, nbytes: int = 256 << 20, repeats: int = 3) -> None:
    """A plain device-to-device copy of `nbytes`, `repeats` times: the reference
    reading for scaling the FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch

    x = torch.ones(nbytes, dtype=torch.uint8, device=device)
    y = torch.empty_like(x)
    for _ in range(repeats):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": nbytes, "repeats": repeats}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (every box here has one GPU)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    PEAKS.update(device_peaks(device))
    if args.only == "copy":
        calibration_copy(device)
        return
    out = {
        "metric": METRIC,
        "value": None,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {},
        "secondary": [],
    }
    if args.only in ("all", "attention"):
        att = bench_attention(args, device)
        out["value"] = att.pop("value")
        out["ms_per_step"] = att.pop("ms_per_step")
        out["config"] = att.pop("config")
        out["roofline"] = att.pop("roofline")
        out["memory"] = att.pop("memory")
        out["kernels"] = att.pop("kernels")
        if "cpu_baseline" in att:
            out["cpu_baseline"] = att.pop("cpu_baseline")
    runs = (("C4", "chunked", lambda: bench_chunked(args, device)),
            ("branch_d256", "fa4_branch", lambda: bench_fa4_branch(args, device)),
            ("C3_gated", "logprob", lambda: bench_logprob(args, device)),
            ("C3_ungated", "logprob_ungated", lambda: bench_logprob(args, device, gate=False)),
            ("rmsnorm", "rmsnorm", lambda: bench_rmsnorm(args, device)),
            ("adjoint", "adjoint", lambda: bench_adjoint(args, device)),
            ("lora", "lora", lambda: bench_lora(args, device)),
            ("C5", "c5", lambda: bench_c5(args, device)))
    for name, only, run in runs:
        if args.only in ("all", only):
            torch.cuda.empty_cache()
            result = run()
            result["name"] = name
            out["secondary"].append(result)
    props = torch.cuda.get_device_properties(device)
    out["device"] = {"name": props.name, "arch": getattr(props, "gcnArchName", ""),
                     "cus": props.multi_processor_count}
    out["peaks"] = dict(PEAKS)
    # the full record first, then the one-line summary the driver reads last
    print(json.dumps({"bench_detail": out}), flush=True)
    print(json.dumps(summary(out), separators=(",", ":")), flush=True)


SECONDARY_FIELDS = ["value", "unit", "ms_per_step", "dominant_kernel", "dominant_frac", "peak_mem_GB",
                    "cpu_baseline", "vs_baseline"]


def summary(out: dict) -> dict:
    """The headline line: the contract's keys, the roofline and CPU baseline of
    the headline workload, and one short row per secondary workload (fields
    in ``secondary.fields``), short enough that a log tail keeps it whole.
    Everything else (per-kernel tables, configs) is in the preceding
    ``bench_detail`` line."""
    keys = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data")
    line = {k: out[k] for k in keys}
    cfg = out.get("config", {})
    line["config"] = {k: cfg[k] for k in ("workload", "visible_pairs", "flop_per_step", "seed") if k in cfg}
    if "roofline" in out:
        line["roofline"] = {k: v for k, v in out["roofline"].items() if k not in ("traffic_source", "work_per_launch")}
    if "cpu_baseline" in out:
        line["cpu_baseline"] = {k: v for k, v in out["cpu_baseline"].items() if k not in ("seconds", "cpu_model")}
    if "memory" in out:
        line["peak_mem_bytes"] = out["memory"]["peak_bytes"]
        line["step_mem_bytes"] = out["memory"]["step_bytes"]
    rows = {"fields": SECONDARY_FIELDS}
    for r in out["secondary"]:
        roof = r.get("roofline") or {}
        cpu = r.get("cpu_baseline") or {}
        mem = r.get("memory") or {}
        kernel = (roof.get("kernel") or "").split(".")[-1].removesuffix("_kernel") or None
        rows[r["name"]] = [r["value"], r["unit"], round(r["ms_per_step"], 3), kernel, roof.get("frac"),
                           round(mem["peak_bytes"] / 1e9, 2) if mem else None, cpu.get("value"),
                           r.get("vs_baseline")]
    line["secondary"] = rows
    line["peaks"] = {k: out["peaks"][k] for k in ("bf16_tflops", "hbm_gbs") if k in out.get("peaks", {})}
    return line


if __name__ == "__main__":
    main()
