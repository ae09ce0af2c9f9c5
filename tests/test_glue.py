"""Host-side glue (CPU): the trial-once capability cache and the operator ranges."""

from __future__ import annotations

import threading
import time

import pytest
import torch

from thundersync_amd import capability, operator_profiling as op


class _FakeCuda:
    """A tensor-like that claims to live on a GPU (the trial never touches it)."""

    def __init__(self, index=0, dtype=torch.bfloat16):
        self.is_cuda = True
        self.device = torch.device("cuda", index)
        self.dtype = dtype


@pytest.fixture
def no_device_calls(monkeypatch):
    """Trials here run no kernel: stand in for the device context and sync."""

    class _Ctx:
        def __init__(self, device):
            pass

        def __enter__(self):
            return None

        def __exit__(self, *exc):
            return False

    monkeypatch.setattr(torch.cuda, "device", _Ctx)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda device=None: None)
    monkeypatch.setattr(capability, "device_identity", lambda device=None: {"index": getattr(device, "index", None)})
    capability.reset_kernel_probes()
    yield
    capability.reset_kernel_probes()


def test_cpu_tensors_never_run_a_trial():
    calls = []
    assert not capability.kernel_runs("k", torch.zeros(1), 0, lambda *a: calls.append(a))
    assert calls == []


def test_trial_runs_once_per_key_with_grad_enabled(no_device_calls):
    calls = []

    def trial(device, dtype, key):
        calls.append((device.index, dtype, key, torch.is_grad_enabled()))

    with torch.no_grad():
        for _ in range(3):
            assert capability.kernel_runs("attn", _FakeCuda(0), 128, trial)
    assert capability.kernel_runs("attn", _FakeCuda(1), 128, trial)
    assert capability.kernel_runs("attn", _FakeCuda(0, torch.float16), 128, trial)
    assert capability.kernel_runs("attn", _FakeCuda(0), 64, trial)
    assert calls == [(0, torch.bfloat16, 128, True), (1, torch.bfloat16, 128, True),
                     (0, torch.float16, 128, True), (0, torch.bfloat16, 64, True)]


def test_failure_is_cached_with_its_error_text(no_device_calls):
    calls = []

    def trial(device, dtype, key):
        calls.append(1)
        raise RuntimeError("no kernel image " + "x" * 1000)

    assert not capability.kernel_runs("bad", _FakeCuda(), 1, trial)
    assert not capability.kernel_runs("bad", _FakeCuda(), 1, trial)
    assert calls == [1]
    (record,) = capability.kernel_probe_records()
    assert record["kernel"] == "bad" and record["runs"] is False and record["shape_key"] == 1
    assert record["dtype"] == "torch.bfloat16" and record["device"] == {"index": 0}
    assert record["error"].startswith("RuntimeError: no kernel image") and len(record["error"]) <= 300


def test_concurrent_callers_of_one_key_share_one_trial(no_device_calls):
    calls, results = [], []

    def slow(device, dtype, key):
        calls.append(1)
        time.sleep(0.2)

    threads = [threading.Thread(target=lambda: results.append(capability.kernel_runs("s", _FakeCuda(), 0, slow)))
               for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert calls == [1] and results == [True] * 4


def test_range_names_and_modes(monkeypatch):
    assert op.range_name("fused_logprob_forward", tokens=3, dtype=torch.bfloat16, skip=None) == \
        "thundersync::fused_logprob_forward|tokens=3|dtype=torch.bfloat16"
    assert op.range_name("x", note="a|b\nc") == "thundersync::x|note=a/b c"
    monkeypatch.setattr(op._State, "mode", None)
    monkeypatch.setenv(op.PROFILE_RANGES_ENV, "NVTX")
    assert op.operator_profiling_mode() == "roctx" and op.operator_profiling_enabled()
    with pytest.raises(ValueError):
        op.configure_operator_profiling("trace")
    op.configure_operator_profiling("off", device_roles={"cpu": "teacher"})
    assert op.device_role("cpu") == "teacher" and op.device_role("cuda:1") == "cuda:1"
    assert op.operator_range("a") is op.operator_range("b")  # the shared do-nothing range
    monkeypatch.setattr(op._State, "mode", None)


def test_kineto_ranges_reach_the_profiler(monkeypatch):
    op.configure_operator_profiling("kineto")
    try:
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
            with op.operator_range("probe_op", rows=7):
                torch.ones(4).sum()
        names = [e.name for e in prof.events()]
        assert "thundersync::probe_op|rows=7" in names
    finally:
        op.configure_operator_profiling("off")
        monkeypatch.setattr(op._State, "mode", None)
