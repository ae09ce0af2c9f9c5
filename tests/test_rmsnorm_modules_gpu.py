"""RMSNorm module swaps on the HIP kernels.

* ``use_stable_qwen3_rms_norm`` (accel/rms_norm.py:55-70 of the reference):
  every Qwen3RMSNorm of a model is replaced, Parameters keep their identity,
  and the forward's bytes equal the stock module's, with and without grad
  (rtol = atol = 0, the reference's tests/test_rms_norm_precision.py:27-39).
* ``use_compiled_source_rms_norm`` (grpo/rms_norm.py:44-84,
  grpo/rms_norm_native.py:98-115): bf16 StableQwen3RMSNorm modules become
  NativeSourceRMSNorm once both trials pass; fp32 modules are left alone; the
  native VJP equals FP32RMSNormVJP's bit for bit (same kernels) and agrees
  with the oracle.
"""

from __future__ import annotations

import pytest
import torch

from oracle import rms_norm as ref

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def tiny_model(device, dtype):
    from transformers import Qwen3Config
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Model

    cfg = Qwen3Config(vocab_size=64, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=32)
    torch.manual_seed(0)
    model = Qwen3Model(cfg).to(device=device, dtype=dtype)
    for m in model.modules():
        if hasattr(m, "variance_epsilon"):
            with torch.no_grad():
                m.weight.copy_(torch.linspace(0.4, 3.0, m.weight.numel()))
    return model


def norms(model):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    return {n: m for n, m in model.named_modules() if isinstance(m, Qwen3RMSNorm)}


def test_stable_swap_keeps_parameters_and_primal(cuda):
    from thundersync_amd.rms_norm import StableQwen3RMSNorm, use_stable_qwen3_rms_norm

    print("stable qwen3 rms norm swap", flush=True)
    model = tiny_model(cuda, torch.bfloat16)
    before = norms(model)
    weights = {n: m.weight for n, m in before.items()}
    x = torch.randn(3, 7, 128, device=cuda, dtype=torch.bfloat16)
    stock = {n: m(x if m.weight.numel() == 128 else x[..., :32]).detach() for n, m in before.items()}
    assert use_stable_qwen3_rms_norm(model) == len(before)
    after = norms(model)
    assert all(isinstance(m, StableQwen3RMSNorm) for m in after.values())
    assert all(after[n].weight is weights[n] for n in after)
    assert use_stable_qwen3_rms_norm(model) == 0
    for n, m in after.items():
        xi = (x if m.weight.numel() == 128 else x[..., :32]).clone().requires_grad_()
        y = m(xi)
        assert y.grad_fn is not None
        assert torch.equal(y.detach(), stock[n])
        with torch.no_grad():
            assert torch.equal(m(xi), stock[n])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("record_graph", [False, True])
@pytest.mark.parametrize("shape", [(64, 128), (3, 7, 4096), (5, 32, 128), (2, 8, 128), (1, 4096), (9, 130)])
def test_stable_vjp_preserves_primal_bytes(cuda, dtype, record_graph, shape):
    """The reference's test_stable_vjp_preserves_primal_bytes (seed 71, linspace
    weights), over its dtypes and grad modes and the C5 norm shapes."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    from thundersync_amd.rms_norm import use_stable_qwen3_rms_norm

    print(f"stable norm primal bytes {shape} {dtype} grad={record_graph}", flush=True)
    torch.manual_seed(71)
    width = shape[-1]
    model = torch.nn.Sequential(Qwen3RMSNorm(width, eps=1e-6)).to(cuda, dtype)
    with torch.no_grad():
        model[0].weight.copy_(torch.linspace(0.4, 3.0, width, device=cuda))
    x = torch.randn(*shape, device=cuda, dtype=dtype)
    with torch.set_grad_enabled(record_graph):
        expected = model(x)
        assert use_stable_qwen3_rms_norm(model) == 1
        torch.testing.assert_close(model(x), expected, rtol=0, atol=0)
    with torch.no_grad():
        no_grad = model(x)
    with torch.enable_grad():
        with_grad = model(x.clone().requires_grad_())
    assert torch.equal(no_grad, with_grad.detach()) and torch.equal(no_grad, expected.detach())


def test_source_swap_and_native_vjp(cuda):
    from thundersync_amd import capability
    from thundersync_amd.rms_norm import FP32RMSNormVJP, use_stable_qwen3_rms_norm
    from thundersync_amd.source_rms_norm import (NativeSourceRMSNorm, native_source_rms_trial,
                                                 use_compiled_source_rms_norm)

    print("source rms norm swap", flush=True)
    capability.reset_kernel_probes()
    native_source_rms_trial(cuda, torch.bfloat16, 128)
    model = tiny_model(cuda, torch.bfloat16)
    use_stable_qwen3_rms_norm(model)
    weights = {n: m.weight for n, m in norms(model).items()}
    assert use_compiled_source_rms_norm(model) == len(weights)
    swapped = norms(model)
    assert all(isinstance(m, NativeSourceRMSNorm) for m in swapped.values())
    assert all(swapped[n].weight is weights[n] for n in swapped)
    records = capability.kernel_probe_records()
    assert {r["kernel"] for r in records} >= {"grpo_source_rms_norm_forward", "grpo_source_rms_norm_native_vjp"}
    assert all(r["runs"] for r in records), records

    norm = next(iter(swapped.values()))
    width = norm.weight.numel()
    g = torch.Generator().manual_seed(3)
    x = torch.randn(129, width, generator=g).to(torch.bfloat16)
    dy = torch.randn(129, width, generator=g).to(torch.bfloat16)
    xa = x.to(cuda).requires_grad_()
    norm.weight.grad = None
    ya = norm(xa)
    ya.backward(dy.to(cuda))
    dw_native = norm.weight.grad.clone()
    xb = x.to(cuda).requires_grad_()
    wb = norm.weight.detach().clone().requires_grad_()
    yb = FP32RMSNormVJP.apply(xb, wb, norm.variance_epsilon)
    yb.backward(dy.to(cuda))
    assert torch.equal(ya, yb) and torch.equal(xa.grad, xb.grad) and torch.equal(dw_native, wb.grad)
    want_dx, want_dw = ref.rms_norm_backward(dy, x, norm.weight.detach().cpu(), norm.variance_epsilon)
    torch.testing.assert_close(xa.grad.cpu().float(), want_dx.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(dw_native.cpu().float(), want_dw.float(), rtol=2e-2, atol=1e-1)


def test_source_swap_skips_fp32(cuda):
    from thundersync_amd.rms_norm import use_stable_qwen3_rms_norm
    from thundersync_amd.source_rms_norm import use_compiled_source_rms_norm

    model = tiny_model(cuda, torch.float32)
    use_stable_qwen3_rms_norm(model)
    assert use_compiled_source_rms_norm(model) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_byte_guard_passes_on_the_device(cuda, dtype):
    """The byte-identity guard's comparison on the device: every row class of
    a 4096-wide and a 128-wide norm reproduces torch's bytes, so the module
    keeps the HIP forward."""
    from thundersync_amd import rms_norm

    print(f"rms norm byte guard {dtype}", flush=True)
    rms_norm.reset_primal_checks()
    g = torch.Generator(device=cuda).manual_seed(9)
    for width in (4096, 128):
        w = torch.linspace(0.4, 3.0, width, device=cuda).to(dtype)
        for rows in (1, 2, 3, 5, 12, 31, 100, 300, 513, 2049):
            x = torch.randn(rows, width, device=cuda, dtype=dtype, generator=g)
            assert rms_norm.hip_takes(x, w)
            assert rms_norm.primal_matches_stock(x, w, 1e-6), (width, rows)
            y, _ = rms_norm.primal_forward(x, w, 1e-6)
            assert torch.equal(y, rms_norm.stock_forward(x, w, 1e-6)[0])
    assert all(rms_norm._MATCHES.values())


def test_swapped_module_takes_stock_forward_for_refused_shapes(cuda):
    """A single row that torch sums across work-groups is refused by the
    kernel; the swapped module then runs the stock forward."""
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    from thundersync_amd import rms_norm

    width = 1 << 18
    model = torch.nn.Sequential(Qwen3RMSNorm(width, eps=1e-6)).to(cuda, torch.bfloat16)
    x = torch.randn(1, width, device=cuda, dtype=torch.bfloat16)
    want = model(x).detach()
    rms_norm.use_stable_qwen3_rms_norm(model)
    assert not rms_norm.hip_takes(x, model[0].weight)
    assert torch.equal(model(x).detach(), want)
