"""The RMSNorm module swap's host logic (CPU, no kernels run).

* The swapped module keeps the stock forward where the reference's module
  does, or where the kernels do not apply (accel/rms_norm.py:49-52): CPU
  tensors in fp32 and bf16, with and without grad, and a weight dtype that
  differs from the hidden dtype.  Outputs and gradients are the stock
  module's, bit for bit.
* The byte-identity guard: the first forward per (device, dtype, width, row
  class) compares the HIP primal with torch's; a planted one-ulp difference
  in the HIP result makes ``auto`` fall back to torch's bytes and
  ``require`` raise.  The HIP forward is replaced by a host stand-in here;
  the real comparison runs on the GPU in tests/test_rmsnorm_modules_gpu.py.
"""

from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm  # noqa: E402

from thundersync_amd import rms_norm  # noqa: E402


def _pair(width, dtype, weight_dtype=None):
    torch.manual_seed(5)
    stock = Qwen3RMSNorm(width, eps=1e-6).to(weight_dtype or dtype)
    with torch.no_grad():
        stock.weight.copy_(torch.linspace(0.4, 3.0, width))
    model = torch.nn.Sequential(Qwen3RMSNorm(width, eps=1e-6).to(weight_dtype or dtype))
    model[0].weight = torch.nn.Parameter(stock.weight.detach().clone())
    assert rms_norm.use_stable_qwen3_rms_norm(model) == 1
    assert isinstance(model[0], rms_norm.StableQwen3RMSNorm)
    return stock, model[0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("grad", [False, True])
def test_cpu_module_is_the_stock_module(dtype, grad):
    stock, swapped = _pair(64, dtype)
    x = torch.randn(3, 5, 64).to(dtype)
    dy = torch.randn(3, 5, 64).to(dtype)
    xa = x.clone().requires_grad_(grad)
    xb = x.clone().requires_grad_(grad)
    with torch.set_grad_enabled(grad):
        ya, yb = stock(xa), swapped(xb)
    assert torch.equal(ya, yb)
    if grad:
        ya.backward(dy)
        yb.backward(dy)
        assert torch.equal(xa.grad, xb.grad)
        assert torch.equal(stock.weight.grad, swapped.weight.grad)


def test_mixed_dtypes_take_the_stock_forward():
    stock, swapped = _pair(32, torch.bfloat16, weight_dtype=torch.float32)
    x = torch.randn(4, 32).to(torch.bfloat16)
    assert not rms_norm.hip_takes(x, swapped.weight)
    assert torch.equal(stock(x), swapped(x))


def test_hip_takes_refuses_host_and_mismatched_calls():
    w = torch.ones(16, dtype=torch.bfloat16)
    assert not rms_norm.hip_takes(torch.zeros(2, 16, dtype=torch.bfloat16), w)
    assert not rms_norm.hip_takes(torch.zeros(2, 16), w)


@pytest.fixture
def host_stand_in(monkeypatch):
    """Run the guard on CPU tensors: the HIP forward becomes torch's ops,
    optionally with the last bit of one primal element flipped."""
    state = {"flip": False}

    def fake_forward(hidden, weight, eps):
        y, rstd = rms_norm.stock_forward(hidden, weight, eps)
        if state["flip"]:
            bits = y.view(torch.int16).clone()
            bits.view(-1)[0] ^= 1
            y = bits.view(y.dtype)
        return y, rstd

    monkeypatch.setattr(rms_norm, "rms_norm_forward", fake_forward)
    monkeypatch.setattr(rms_norm, "_check_device", lambda h, w: None)
    rms_norm.reset_primal_checks()
    yield state
    rms_norm.reset_primal_checks()


def test_guard_accepts_equal_bytes(host_stand_in, monkeypatch):
    monkeypatch.setattr(rms_norm._lib, "resolved_setting", lambda: "auto")
    x = torch.randn(7, 48).to(torch.bfloat16)
    w = torch.linspace(0.5, 2.0, 48).to(torch.bfloat16)
    assert rms_norm.primal_matches_stock(x, w, 1e-6)
    y, _ = rms_norm.primal_forward(x, w, 1e-6)
    assert torch.equal(y, rms_norm.stock_forward(x, w, 1e-6)[0])


def test_guard_falls_back_under_auto(host_stand_in, monkeypatch):
    monkeypatch.setattr(rms_norm._lib, "resolved_setting", lambda: "auto")
    host_stand_in["flip"] = True
    x = torch.randn(7, 48).to(torch.bfloat16)
    w = torch.linspace(0.5, 2.0, 48).to(torch.bfloat16)
    assert not rms_norm.primal_matches_stock(x, w, 1e-6)
    y, rstd = rms_norm.primal_forward(x, w, 1e-6)
    want_y, want_rstd = rms_norm.stock_forward(x, w, 1e-6)
    assert torch.equal(y, want_y) and torch.equal(rstd, want_rstd)
    # the decision is per row class: 7 rows (class 4) and 2 rows (class 2) differ
    host_stand_in["flip"] = False
    assert rms_norm.primal_matches_stock(x[:2], w, 1e-6)
    assert not rms_norm.primal_matches_stock(x[:5], w, 1e-6)  # class 4, cached


def test_guard_raises_under_require(host_stand_in, monkeypatch):
    monkeypatch.setattr(rms_norm._lib, "resolved_setting", lambda: "require")
    host_stand_in["flip"] = True
    x = torch.randn(3, 48).to(torch.bfloat16)
    w = torch.ones(48, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="differs from torch's RMSNorm bytes"):
        rms_norm.primal_matches_stock(x, w, 1e-6)


def test_row_classes_follow_torchs_schedule():
    assert [rms_norm._row_class(n) for n in (1, 2, 3, 7, 8, 511, 512, 513, 10**6)] == [
        1, 2, 2, 4, 8, 256, 512, 512, 512]
