"""HIP merged-weight LoRA linear against the CPU oracle (accel/fused_lora.py:26-48).

Bars (max-abs over max|oracle|, printed with the absolute max-abs):
* y and dx (bf16 outputs of fp32 sums over bf16 inputs): 1e-2;
* dA and dB (fp32 sums over the bf16-rounded rank products g B and x A^T,
  as the device forms them): 2e-3 against the oracle that rounds them the
  same way, 2e-2 against the unrounded one.
The module test repeats the reference's gate (tests/test_fused_lora.py:39-70)
with a bf16 base on the GPU against the fp32 unmerged layer on the CPU.
"""

from __future__ import annotations

import pytest
import torch

from oracle import lora as ref
from thundersync_amd import fused_lora
from thundersync_amd.lora_layers import LoraLinear, add_lora

pytestmark = pytest.mark.gpu


def close(got, want, bar, what):
    got, want = got.detach().double().cpu(), want.detach().double().cpu()
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = (got - want).abs().max().item() if got.numel() else 0.0
    scale = max(want.abs().max().item() if want.numel() else 0.0, 1e-6)
    print(f"  {what}: max-abs {err:.3g} (bar {bar} x {scale:.3g})", flush=True)
    assert err <= bar * scale, f"{what}: max-abs {err:.3g} > {bar} x {scale:.3g}"


def _inputs(rows, inp, out, rank, seed, adapter_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, inp, generator=g).to(torch.bfloat16)
    w = (torch.randn(out, inp, generator=g) * inp ** -0.5).to(torch.bfloat16)
    a = (torch.randn(rank, inp, generator=g) * inp ** -0.5).to(adapter_dtype)
    b = (torch.randn(out, rank, generator=g) * 0.1).to(adapter_dtype)
    dy = torch.randn(rows, out, generator=g).to(torch.bfloat16)
    return x, w, a, b, dy


def run(cuda, x, w, a, b, dy, scale, *, x_grad=True):
    xc = x.to(cuda).requires_grad_(x_grad)
    ac, bc = a.to(cuda).requires_grad_(), b.to(cuda).requires_grad_()
    y = fused_lora.FusedLoRALinear.apply(xc, w.to(cuda), ac, bc, scale)
    y.backward(dy.to(cuda))
    torch.cuda.synchronize()
    return y, xc.grad, ac.grad, bc.grad


SHAPES = [
    # rows, in, out, rank
    (300, 256, 512, 16),
    (1, 64, 128, 8),
    (5, 128, 64, 4),
    (1000, 512, 1024, 64),
    (777, 1024, 256, 1),
    (513, 256, 264, 256),
    (4096, 4096, 1024, 16),  # C5 k/v projection, one 4096-token slice
]


@pytest.mark.parametrize("rows,inp,out,rank", SHAPES)
def test_matches_oracle(cuda, rows, inp, out, rank):
    print(f"lora rows={rows} in={inp} out={out} rank={rank}", flush=True)
    x, w, a, b, dy = _inputs(rows, inp, out, rank, seed=rows + inp + rank)
    scale = 2.0
    y, dx, da, db = run(cuda, x, w, a, b, dy, scale)
    assert y.dtype == torch.bfloat16 and dx.dtype == torch.bfloat16
    assert da.dtype == torch.float32 and db.dtype == torch.float32
    close(y, ref.fused_forward(x, w), 1e-2, "y")
    want_dx, want_da, want_db = ref.fused_backward(dy, x, w, a.to(torch.bfloat16), b.to(torch.bfloat16), scale,
                                                   round_rank=True)
    close(dx, want_dx, 1e-2, "dx")
    close(da, want_da, 2e-3, "dA (rank products rounded)")
    close(db, want_db, 2e-3, "dB (rank products rounded)")
    _, exact_da, exact_db = ref.fused_backward(dy, x, w, a.to(torch.bfloat16), b.to(torch.bfloat16), scale)
    close(da, exact_da, 2e-2, "dA")
    close(db, exact_db, 2e-2, "dB")


def test_batched_strided_input_and_adapter_dtypes(cuda):
    print("lora 3-d strided x, bf16 adapters, frozen x", flush=True)
    g = torch.Generator().manual_seed(9)
    wide = torch.randn(2, 70, 192, generator=g).to(torch.bfloat16)
    x = wide[..., :128]  # row stride 192
    w = (torch.randn(96, 128, generator=g) * 0.1).to(torch.bfloat16)
    a = (torch.randn(8, 128, generator=g) * 0.1).to(torch.bfloat16)
    b = (torch.randn(96, 8, generator=g) * 0.1).to(torch.bfloat16)
    dy = torch.randn(2, 70, 96, generator=g).to(torch.bfloat16)
    y, dx, da, db = run(cuda, x, w, a, b, dy, 0.5, x_grad=False)
    assert y.shape == (2, 70, 96) and dx is None
    assert da.dtype == torch.bfloat16 and db.dtype == torch.bfloat16
    x2, dy2 = x.reshape(-1, 128), dy.reshape(-1, 96)
    close(y.reshape(-1, 96), ref.fused_forward(x2, w), 1e-2, "y")
    _, want_da, want_db = ref.fused_backward(dy2, x2, w, a, b, 0.5, round_rank=True)
    close(da, want_da, 1e-2, "dA")
    close(db, want_db, 1e-2, "dB")


def test_no_rows_gives_zero_adapter_gradients(cuda):
    x, w, a, b, dy = _inputs(0, 64, 64, 4, seed=1)
    y, dx, da, db = run(cuda, x, w, a, b, dy, 1.0)
    assert y.shape == (0, 64) and dx.shape == (0, 64)
    assert torch.count_nonzero(da) == 0 and torch.count_nonzero(db) == 0


def test_repeated_backward_is_bit_identical(cuda):
    x, w, a, b, dy = _inputs(3000, 512, 256, 16, seed=4)
    first = run(cuda, x, w, a, b, dy, 2.0)
    second = run(cuda, x, w, a, b, dy, 2.0)
    for f, s in zip(first, second):
        assert torch.equal(f, s)


def test_module_gate_against_the_unmerged_layer(cuda):
    """tests/test_fused_lora.py:39-70 on the GPU: a bf16 two-layer model with
    fp32 adapters, fused, against the unmerged fp32 model on the CPU."""
    torch.manual_seed(11)
    base = torch.nn.Sequential()
    base.add_module("up", torch.nn.Linear(256, 512, bias=False))
    base.add_module("act", torch.nn.Tanh())
    base.add_module("down", torch.nn.Linear(512, 256, bias=False))
    add_lora(base, ["up", "down"], rank=16, alpha=32)
    for layer in base.modules():
        if isinstance(layer, LoraLinear):
            torch.nn.init.normal_(layer.lora_B["default"].weight, std=0.05)
    reference = base
    candidate = torch.nn.Sequential()
    candidate.add_module("up", torch.nn.Linear(256, 512, bias=False))
    candidate.add_module("act", torch.nn.Tanh())
    candidate.add_module("down", torch.nn.Linear(512, 256, bias=False))
    add_lora(candidate, ["up", "down"], rank=16, alpha=32)
    candidate.load_state_dict(reference.state_dict())
    for layer in candidate.modules():
        if isinstance(layer, LoraLinear):
            layer.base_layer.to(cuda, torch.bfloat16)
            layer.lora_A.to(cuda)
            layer.lora_B.to(cuda)
    x = torch.randn(300, 256)

    def grads(model, inp):
        for p in model.parameters():
            p.grad = None
        out = model(inp)
        out.float().pow(2).sum().backward()
        return out.detach(), {n: p.grad.detach() for n, p in model.named_parameters() if p.grad is not None}

    # the reference side sees the same bf16-rounded base weights
    with torch.no_grad():
        for layer in reference.modules():
            if isinstance(layer, LoraLinear):
                layer.base_layer.weight.copy_(layer.base_layer.weight.to(torch.bfloat16).float())
    want_out, want = grads(reference, x.to(torch.bfloat16).float())
    assert fused_lora.fuse_merged_lora_forward(candidate) == 2
    got_out, got = grads(candidate, x.to(cuda, torch.bfloat16))
    assert set(got) == set(want) and len(got) == 4
    close(got_out, want_out, 2e-2, "model output")
    for name in want:
        assert got[name].dtype == torch.float32
        close(got[name], want[name], 3e-2, name)
    assert fused_lora.unfuse_merged_lora_forward(candidate) == 2
