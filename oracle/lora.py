"""CPU restatement of the reference's merged-weight LoRA linear -- TEST
INFRASTRUCTURE ONLY (the parity tests' checker; the product never imports it).

* :func:`fused_forward` -- accel/fused_lora.py:29-33: ``x @ W_eff.T``.
* :func:`fused_backward` -- accel/fused_lora.py:35-48: ``dx = g W_eff``,
  ``dA = s (g B)^T x``, ``dB = s g^T (x A^T)``, computed here in fp64 from
  the given values (optionally rounding ``g B`` and ``x A^T`` to bf16 first,
  the operands the device forms them as).
* :func:`unfused_forward` -- the expression the fused layer replaces (PEFT's
  LoRA linear without dropout): ``x W^T + s (x A^T) B^T``.

Pinned in tests/test_oracle_lora.py: the fused backward equals fp64 autograd
of :func:`unfused_forward` (the reference's claim that the fused gradients
are the exact derivative, tests/test_fused_lora.py:39-70), and the fused
forward over ``W + s B A`` equals the unfused value.
"""

from __future__ import annotations

import torch


def merged_weight(weight: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor, scaling: float) -> torch.Tensor:
    """``W + s B A`` in fp64."""
    return weight.double() + scaling * (lora_b.double() @ lora_a.double())


def fused_forward(x: torch.Tensor, weight_eff: torch.Tensor) -> torch.Tensor:
    """accel/fused_lora.py:32-33, fp64."""
    return x.double() @ weight_eff.double().t()


def unfused_forward(x, weight, lora_a, lora_b, scaling):
    """``x W^T + s (x A^T) B^T``, fp64 (autograd-capable)."""
    return x @ weight.t() + scaling * ((x @ lora_a.t()) @ lora_b.t())


def fused_backward(grad_out, x, weight_eff, lora_a, lora_b, scaling, *, round_rank: bool = False):
    """accel/fused_lora.py:35-48 in fp64: (dx, dA, dB).  With ``round_rank`` the
    rank-sized products ``g B`` and ``x A^T`` are rounded to bf16 before use.
    ``weight_eff`` None skips dx (returned as None)."""
    g, xx = grad_out.double(), x.double()
    a, b = lora_a.double(), lora_b.double()
    u = g @ b
    t = xx @ a.t()
    if round_rank:
        u = u.to(torch.bfloat16).double()
        t = t.to(torch.bfloat16).double()
    dx = None if weight_eff is None else g @ weight_eff.double()
    da = scaling * (u.t() @ xx)
    db = scaling * (g.t() @ t)
    return dx, da, db


def reference_step(x, weight, lora_a, lora_b, grad_out, scaling):
    """The reference layer's forward and backward as its own code computes them
    (accel/fused_lora.py:32-47: products in the activation dtype, the scale
    applied after, gradients cast to each adapter's dtype): the eager CPU path
    bench.py times as the baseline.  Returns (y, dx, dA, dB)."""
    y = x @ weight.t()
    a, b = lora_a.to(x.dtype), lora_b.to(x.dtype)
    dx = grad_out @ weight
    da = ((grad_out @ b).transpose(-2, -1) @ x * scaling).to(lora_a.dtype)
    db = (grad_out.transpose(-2, -1) @ (x @ a.t()) * scaling).to(lora_b.dtype)
    return y, dx, da, db
