"""THUNDERSYNC_HIP = require | off | auto, with THUNDERSYNC_FA4's semantics.

Mirrors the reference's switch tests (tests/test_fa4_switch.py:36-62): `off`
never loads, `require` raises at every resolution while the library cannot
load, `auto` leaves the path absent, unknown settings are refused.
"""

from __future__ import annotations

import pytest

from thundersync_amd import _lib


@pytest.fixture
def unresolved(monkeypatch):
    _lib.reset()
    yield
    _lib.reset()


def test_off_never_loads(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "off")
    called = []
    monkeypatch.setattr(_lib, "_load", lambda: called.append(1))
    assert _lib.library() is None
    assert _lib.hip_build() is None
    assert called == []
    with pytest.raises(RuntimeError, match="switched off"):
        _lib.require_library()


def test_require_without_a_library_raises_every_time(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "require")

    def missing():
        raise OSError("not built")

    monkeypatch.setattr(_lib, "_load", missing)
    for _ in range(2):
        with pytest.raises(RuntimeError, match="THUNDERSYNC_HIP=require"):
            _lib.library()
    assert _lib._RESOLVED is False
    assert _lib.hip_build() is None


def test_auto_without_a_library_leaves_it_absent(unresolved, monkeypatch):
    monkeypatch.delenv(_lib.HIP_ENV, raising=False)

    def missing():
        raise OSError("not built")

    monkeypatch.setattr(_lib, "_load", missing)
    assert _lib.hip_setting() == "auto"
    assert _lib.library() is None
    assert _lib._RESOLVED is True
    with pytest.raises(RuntimeError, match="not available"):
        _lib.require_library()


def test_an_unknown_setting_is_refused(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "maybe")
    with pytest.raises(ValueError, match="THUNDERSYNC_HIP"):
        _lib.library()


def test_require_with_the_library_resolves_once(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "require")
    lib = _lib.library()
    assert lib is not None and _lib.library() is lib
    assert _lib.hip_build().startswith("thundersync_hip")


# -- trial-gated dispatch and path counters (engine/streaming.py:355-373, 532-548) --

class _FakeCuda:
    def __init__(self, dtype, head_dim=128, index=0):
        import torch

        self.is_cuda = True
        self.dtype = dtype
        self.device = torch.device("cuda", index)
        self.shape = (1, 4, 8, head_dim)


@pytest.fixture
def trial_recorder(monkeypatch):
    from thundersync_amd import capability, dispatch

    calls = []

    def fake_runs(kernel, like, key, trial):
        calls.append((kernel, like.device.index, str(like.dtype), key))
        return like.device.index != 1  # "device 1" fails its trial

    monkeypatch.setattr(dispatch, "kernel_runs", fake_runs)
    capability.reset_kernel_probes()
    return calls


def test_auto_takes_the_kernels_only_after_a_device_trial(unresolved, monkeypatch, trial_recorder):
    import torch

    from thundersync_amd import dispatch

    monkeypatch.delenv(_lib.HIP_ENV, raising=False)
    assert dispatch.hip_attention_available(_FakeCuda(torch.bfloat16))
    assert trial_recorder == [("hip_attention", 0, "torch.bfloat16", 128)]
    assert not dispatch.hip_attention_available(_FakeCuda(torch.bfloat16, index=1))
    # fp16 and every head dim take their own trial; fp32 never reaches one
    assert dispatch.hip_attention_available(_FakeCuda(torch.float16))
    assert trial_recorder[-1] == ("hip_attention", 0, "torch.float16", 128)
    assert not dispatch.hip_attention_available(_FakeCuda(torch.float32))
    assert dispatch.hip_attention_available(_FakeCuda(torch.bfloat16, head_dim=256))
    assert trial_recorder[-1] == ("hip_attention", 0, "torch.bfloat16", 256)
    # a head dim the kernels are not built for runs zero-padded (its own
    # trial); above 256 none runs
    assert dispatch.hip_attention_available(_FakeCuda(torch.bfloat16, head_dim=80))
    assert trial_recorder[-1] == ("hip_attention", 0, "torch.bfloat16", 80)
    assert not dispatch.hip_attention_available(_FakeCuda(torch.bfloat16, head_dim=320))
    assert len(trial_recorder) == 5
    assert dispatch.hip_logprob_available(_FakeCuda(torch.bfloat16))
    assert trial_recorder[-1] == ("hip_logprob", 0, "torch.bfloat16", 128)
    # the fused logprob also takes fp32 and fp64 (its input-precision kernels)
    assert dispatch.hip_logprob_available(_FakeCuda(torch.float32))
    assert trial_recorder[-1] == ("hip_logprob", 0, "torch.float32", 128)
    assert dispatch.hip_logprob_available(_FakeCuda(torch.float64))
    assert not dispatch.hip_logprob_available(_FakeCuda(torch.int32))


def test_require_skips_the_trial_and_off_never_loads(unresolved, monkeypatch, trial_recorder):
    import torch

    from thundersync_amd import dispatch

    monkeypatch.setenv(_lib.HIP_ENV, "require")
    assert dispatch.hip_attention_available(_FakeCuda(torch.bfloat16, index=1))
    assert trial_recorder == []
    _lib.reset()
    monkeypatch.setenv(_lib.HIP_ENV, "off")
    monkeypatch.setattr(_lib, "_load", lambda: (_ for _ in ()).throw(AssertionError("loaded")))
    assert not dispatch.hip_attention_available(_FakeCuda(torch.bfloat16))
    assert trial_recorder == []


def test_require_without_a_library_raises_at_the_dispatch(unresolved, monkeypatch, trial_recorder):
    import torch

    from thundersync_amd import dispatch

    monkeypatch.setenv(_lib.HIP_ENV, "require")
    monkeypatch.setattr(_lib, "_load", lambda: (_ for _ in ()).throw(OSError("not built")))
    for _ in range(2):
        with pytest.raises(RuntimeError, match="THUNDERSYNC_HIP=require"):
            dispatch.hip_attention_available(_FakeCuda(torch.bfloat16))


def test_attention_path_counts_are_cumulative_and_thread_safe():
    import threading

    from thundersync_amd import dispatch

    dispatch.reset_attention_path_counts()
    threads = [threading.Thread(target=lambda: [dispatch.count_attention_path("hip") for _ in range(500)])
               for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    dispatch.count_attention_path("hip_backward", 3)
    assert dispatch.attention_path_counts() == {"hip": 2000, "hip_backward": 3}
    dispatch.reset_attention_path_counts()
