"""The LoRA oracle against fp64 autograd of the unmerged layer (CPU).

The reference's claim (tests/test_fused_lora.py:39-70): the fused layer's
forward over the merged weight is the unmerged layer's value, and its
hand-written gradients are the exact derivative of the unmerged expression.
Checked here in fp64 with autograd as the independent side, over ranks and
scalings, so that a transposed operand, a dropped scale or a swapped
adapter in the oracle fails.
"""

from __future__ import annotations

import pytest
import torch

from oracle import lora as ref


@pytest.mark.parametrize("rows,inp,out,rank,scale", [(7, 16, 24, 4, 2.0), (32, 64, 128, 8, 0.5), (5, 8, 8, 1, 3.0)])
def test_fused_gradients_are_the_unmerged_derivative(rows, inp, out, rank, scale):
    g = torch.Generator().manual_seed(rows + inp + rank)
    x = torch.randn(rows, inp, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(out, inp, generator=g, dtype=torch.float64)
    a = torch.randn(rank, inp, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(out, rank, generator=g, dtype=torch.float64, requires_grad=True)
    dy = torch.randn(rows, out, generator=g, dtype=torch.float64)
    y = ref.unfused_forward(x, w, a, b, scale)
    want_dx, want_da, want_db = torch.autograd.grad(y, (x, a, b), dy)
    w_eff = ref.merged_weight(w, a.detach(), b.detach(), scale)
    torch.testing.assert_close(ref.fused_forward(x.detach(), w_eff), y.detach(), rtol=1e-12, atol=1e-12)
    dx, da, db = ref.fused_backward(dy, x.detach(), w_eff, a.detach(), b.detach(), scale)
    torch.testing.assert_close(dx, want_dx, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(da, want_da, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(db, want_db, rtol=1e-12, atol=1e-12)
    assert da.shape == (rank, inp) and db.shape == (out, rank)


def test_rank_rounding_only_moves_adapter_gradients():
    g = torch.Generator().manual_seed(3)
    x, dy = torch.randn(40, 32, generator=g), torch.randn(40, 16, generator=g)
    w, a, b = torch.randn(16, 32, generator=g), torch.randn(4, 32, generator=g), torch.randn(16, 4, generator=g)
    exact = ref.fused_backward(dy, x, w, a, b, 2.0)
    rounded = ref.fused_backward(dy, x, w, a, b, 2.0, round_rank=True)
    assert torch.equal(exact[0], rounded[0])
    for e, r in zip(exact[1:], rounded[1:]):
        assert not torch.equal(e, r)
        torch.testing.assert_close(r, e, rtol=2e-2, atol=2e-2 * e.abs().max().item())


def test_reference_step_agrees_with_the_fp64_restatement():
    g = torch.Generator().manual_seed(8)
    x, dy = torch.randn(33, 48, generator=g), torch.randn(33, 40, generator=g)
    w, a, b = torch.randn(40, 48, generator=g), torch.randn(6, 48, generator=g), torch.randn(40, 6, generator=g)
    y, dx, da, db = ref.reference_step(x, w, a, b, dy, 1.5)
    want = ref.fused_backward(dy, x, w, a, b, 1.5)
    torch.testing.assert_close(y.double(), ref.fused_forward(x, w), rtol=1e-5, atol=1e-4)
    for got, exp in zip((dx, da, db), want):
        torch.testing.assert_close(got.double(), exp, rtol=1e-5, atol=1e-4)
