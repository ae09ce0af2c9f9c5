"""RMSNorm oracle (CPU).

Restates accel/rms_norm.py:9-17 (forward: ``x = h.float(); rstd =
rsqrt(mean(x^2) + eps); y = w * (x * rstd).to(dtype)``) and the FP32 VJP of
accel/rms_norm.py:33-38 (autograd of ``F.rms_norm`` in fp32 on the CPU).

Pinned by: the forward against transformers' stock ``Qwen3RMSNorm`` (bytes
equal, the reference's own claim, tests/test_rms_norm_precision.py:27-39);
the VJP against an fp64 autograd of the unrounded formula and against the
closed form ``dx = rstd*(g - xhat*mean(g*xhat))``, ``dw = sum(dy*xhat)``.
"""

from __future__ import annotations

import torch


def rms_norm_forward(hidden: torch.Tensor, weight: torch.Tensor, eps: float):
    """accel/rms_norm.py:11-14. Returns (primal, rstd[..., 1] fp32)."""
    x = hidden.to(torch.float32)
    variance = x.pow(2).mean(-1, keepdim=True)
    rstd = torch.rsqrt(variance + eps)
    primal = weight * (x * rstd).to(hidden.dtype)
    return primal, rstd


def rms_norm_backward(gradient, hidden, weight, eps: float):
    """accel/rms_norm.py:33-38: autograd of F.rms_norm in fp32.

    Returns (dx in hidden.dtype, dw in weight.dtype).
    """
    with torch.enable_grad():
        x = hidden.detach().float().requires_grad_()
        w = weight.detach().float().requires_grad_()
        out = torch.nn.functional.rms_norm(x, tuple(weight.shape), w, eps)
        dx, dw = torch.autograd.grad(out, (x, w), gradient.float())
    return dx.to(hidden.dtype), dw.to(weight.dtype)


def rms_norm_backward_closed_form(gradient, hidden, weight, rstd):
    """The VJP written out, in fp64, from the saved statistic (for pinning)."""
    x = hidden.double()
    r = rstd.double()
    g = gradient.double() * weight.double()
    xhat = x * r
    dot = (g * xhat).mean(-1, keepdim=True)
    dx = r * (g - xhat * dot)
    dw = (gradient.double() * xhat).reshape(-1, hidden.shape[-1]).sum(0)
    return dx, dw
