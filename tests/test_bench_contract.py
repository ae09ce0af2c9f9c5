"""bench.py's host-side contract (CPU): the one-GPU guard, the roofline
arithmetic, the traffic table lookup and the CPU-baseline repetition helper."""

from __future__ import annotations

import json
import subprocess
import sys

import pytest

from tests.conftest import ROOT

sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused_with_a_message():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=60)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr and proc.stdout == ""


def test_roofline_of_picks_the_kernel_with_the_largest_device_time():
    per = {"a": (1.0, 1.0), "b": (0.5, 3.0)}  # b: 1.5 ms per step
    roof = bench.roofline_of(per, {"a": 1e12, "b": 6e12}, "TFLOP/s", 2500.0, "no-such-workload")
    assert roof["kernel"] == "b" and roof["bound"] == "mfma"
    assert roof["work_per_launch"] == pytest.approx(2e12)
    assert roof["achieved"] == pytest.approx(2e12 / 0.5e-3 / 1e12)  # 4000 TFLOP/s
    assert roof["frac"] == pytest.approx(roof["achieved"] / 2500.0, rel=1e-3)
    assert roof["traffic"] is None and roof["traffic_source"] is None
    hbm = bench.roofline_of({"c": (0.1, 1.0)}, {"c": 4e8}, "GB/s", 8000.0, "no-such-workload")
    assert hbm["bound"] == "hbm" and hbm["achieved"] == pytest.approx(4000.0)


def test_traffic_table_entries_name_their_commit():
    table = json.loads((ROOT / "profiles" / "traffic.json").read_text())
    for workload, kernels in table["workloads"].items():
        for kernel, entry in kernels.items():
            got = bench.measured_entry(workload, kernel)
            assert abs(got["traffic_bytes"] - (entry["fetch_bytes"] + entry["write_bytes"])) <= 1  # rounding
            assert got["measured_at_commit"] and len(got["measured_at_commit"]) >= 7


def test_summary_line_keeps_every_secondary_in_a_short_line(monkeypatch):
    """The summary line (the driver reads the last 2000 characters of the
    output) carries the contract's keys, the roofline and CPU baseline, and
    one row per secondary workload."""
    out = {k: 1 for k in ("value", "n_gpus", "steps", "warmup", "ms_per_step")}
    out.update(metric=bench.METRIC, unit="TFLOP/s", higher_is_better=True, scaling="weak", vs_baseline=None,
               dtype="bf16", data="synthetic",
               config={"workload": "C2 forest attention fwd+bwd: 2048-token shared prompt + 8 completions "
                                   "U[256,4096], 32/8 heads, head_dim 128, bf16", "visible_pairs": 71374048,
                       "flop_per_step": 4092873408512, "seed": 0, "completion_lengths": list(range(8))},
               roofline={"kernel": "attention.dkdv_kernel", "bound": "mfma", "achieved": 844.39, "peak": 2516.6,
                         "unit": "TFLOP/s", "frac": 0.3355, "traffic": 12655191624, "avg_launch_ms": 2.7698,
                         "launches_per_step": 1.0, "traffic_source": "x" * 80, "work_per_launch": 2.3e12,
                         "sustained_clock_mhz": 2100, "frac_at_sustained_clock": 0.3834},
               cpu_baseline={"value": 1.0852, "unit": "TFLOP/s", "cores": 16, "cpu_model": "AMD EPYC 9575F",
                             "kind": "port", "seconds": 10.5,
                             "sample": "prompt node (2048 rows) + first completion node (2943 rows) of the "
                                       "same C2 forest, 12457536 visible pairs, fp32 masked S"},
               memory={"resident_bytes": 10 ** 9, "peak_bytes": 6123456789, "step_bytes": 5123456789},
               peaks={"bf16_tflops": 2516.6, "hbm_gbs": 8000.0, "clock_mhz": 2400.0},
               kernels={"k%d" % i: {"avg_ms": 1.0} for i in range(40)})
    names = ["C4", "branch_d256", "C3_gated", "C3_ungated", "rmsnorm", "adjoint", "lora", "C5"]
    out["secondary"] = [{"name": n, "value": 123456.78, "unit": "tokens/s", "ms_per_step": 57.59123,
                         "roofline": {"kernel": "logprob.grad_hidden_reduce_kernel", "frac": 0.3123},
                         "memory": {"peak_bytes": 60123456789}, "cpu_baseline": {"value": 1.1412},
                         "kernels": {"k%d" % i: {"avg_ms": 1.0} for i in range(20)}} for n in names]
    line = json.dumps(bench.summary(out), separators=(",", ":"))
    assert len(line) < 1900, len(line)
    back = json.loads(line)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in back, key
    assert set(back["secondary"]) == {"fields", *names}
    assert len(back["secondary"]["C4"]) == len(back["secondary"]["fields"])
    assert back["peak_mem_bytes"] == 6123456789


def test_repeat_for_runs_at_least_once_and_stops():
    calls = []
    reps, dt = bench.repeat_for(lambda: calls.append(1), seconds=0.0)
    assert reps == 1 and len(calls) == 1 and dt >= 0.0
    reps, _ = bench.repeat_for(lambda: None, seconds=100.0, max_reps=7)
    assert reps == 7


def test_cpu_baseline_uses_every_affinity_core_and_names_the_cpu():
    import os

    assert bench.cpu_threads() == len(os.sched_getaffinity(0))
    model = bench.cpu_model()
    assert isinstance(model, str) and model


def test_mfma_peak_follows_cus_and_clock(monkeypatch):
    import torch

    from thundersync_amd import _lib

    monkeypatch.setattr(_lib, "device_clocks",
                        lambda i: {"cus": 256, "clock_khz": 2_400_000, "mem_clock_khz": 2_000_000,
                                   "mem_bus_bits": 8192})
    peaks = bench.device_peaks(torch.device("cuda", 0))
    # 256 CUs x 2.4 GHz x 4096 FLOP per CU per clock: the published 2.5 PFLOP/s
    assert peaks["bf16_tflops"] == pytest.approx(2516.6, abs=0.1)
    assert peaks["cus"] == 256 and peaks["clock_mhz"] == 2400.0 and peaks["hbm_gbs"] == 8000.0
