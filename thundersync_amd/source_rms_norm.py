"""GRPO source RMSNorm on the gfx950 kernels.

The reference's GRPO path swaps bf16 ``StableQwen3RMSNorm`` modules in two
steps, each adopted only once a trial passes on the device
(grpo/rms_norm.py:44-84, grpo/rms_norm_native.py:49-115): a forward whose
reduction Inductor compiles, then a native VJP (aten's dx with Triton dW
schedules, adopted only if bitwise equal to aten's fused FP32 VJP).  In this
build both are the library's kernels, which ``StableQwen3RMSNorm`` already
runs: ``ts_rmsnorm_fwd`` (bytes equal to the stock module's) and
``ts_rmsnorm_bwd`` (the FP32 VJP from the saved statistic, dW summed in a
fixed order).  :func:`use_compiled_source_rms_norm` keeps the reference's
contract -- names, the per-width trial keys ``grpo_source_rms_norm_forward``
and ``grpo_source_rms_norm_native_vjp``, bf16 modules only, Parameters kept,
a module whose trials fail left as it is -- and marks the modules whose
trials passed as :class:`NativeSourceRMSNorm`.

The trials are this build's own:

* forward: for inputs shaped ``(1, 3, W)`` and ``(1, 3, 2, W)`` the HIP
  primal equals torch's stock operations on the device byte for byte, and
  the VJP is finite;
* native VJP: two runs give the same bits, and dx and dW agree with the FP32
  closed form computed by torch operations on the device within the bf16
  rounding of the stored results, over 3, 129 and 65537 rows.

Not bitwise against aten: the reference's bitwise trial compares aten's
fused backward with Triton schedules written to reproduce its summation
order; that order is not available in this image (torch ships the kernel's
header, not its source), and this build's dW has its own fixed order.
"""

from __future__ import annotations

import torch

from .capability import kernel_runs
from .rms_norm import rms_norm_backward, rms_norm_forward

try:
    from .rms_norm import StableQwen3RMSNorm, replace_norms
except ImportError:  # pragma: no cover - transformers absent
    StableQwen3RMSNorm = None

FORWARD_TRIAL = "grpo_source_rms_norm_forward"
NATIVE_VJP_TRIAL = "grpo_source_rms_norm_native_vjp"


def native_source_rms_backward(gradient, hidden, weight, rstd, needs=(True, True)):
    """``(dx, dw)`` of the FP32 VJP from the saved ``rstd``, each None when not
    needed (grpo/rms_norm_native.py:49-75's signature)."""
    with torch.autocast(device_type=hidden.device.type, enabled=False):
        return rms_norm_backward(gradient.contiguous(), hidden, weight, rstd, tuple(needs))


def compiled_source_rms_trial(device, dtype, width, eps=1e-6):
    """Raise unless the HIP forward reproduces the stock bytes and its VJP is finite."""
    g = torch.Generator(device=device).manual_seed(71)
    weight = torch.linspace(0.4, 3.0, width, device=device, dtype=dtype)
    for shape in ((1, 3, width), (1, 3, 2, width)):
        hidden = torch.randn(shape, device=device, dtype=dtype, generator=g)
        primal, rstd = rms_norm_forward(hidden, weight, eps)
        x = hidden.float()
        stock = weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)).to(dtype)
        if not torch.equal(primal, stock):
            raise RuntimeError("source RMSNorm forward differs from the stock module's bytes")
        dx, dw = native_source_rms_backward(torch.ones_like(hidden), hidden, weight, rstd)
        if not (dx.isfinite().all() and dw.isfinite().all()):
            raise RuntimeError("source RMSNorm VJP produced nonfinite values")


def native_source_rms_trial(device, dtype, width):
    """Raise unless the native VJP is reproducible and agrees with the FP32
    closed form on the device (rows 3, 129, 65537, as the reference tries)."""
    g = torch.Generator(device=device).manual_seed(710)
    weight = torch.linspace(0.4, 3.0, width, device=device, dtype=dtype)
    ulp = torch.finfo(dtype).eps
    for rows in (3, 129, 65537):
        hidden = torch.randn(rows, width, device=device, dtype=dtype, generator=g)
        gradient = torch.randn(rows, width, device=device, dtype=dtype, generator=g)
        rstd = torch.rsqrt(hidden.float().square().mean(-1, keepdim=True) + 1e-6)
        first = native_source_rms_backward(gradient, hidden, weight, rstd)
        again = native_source_rms_backward(gradient, hidden, weight, rstd)
        if not all(torch.equal(a, b) for a, b in zip(first, again)):
            raise RuntimeError("native source RMSNorm VJP is not reproducible")
        xhat = hidden.float() * rstd
        gw = gradient.float() * weight.float()
        dx = rstd * (gw - xhat * (gw * xhat).mean(-1, keepdim=True))
        dw = (gradient.float() * xhat).sum(0)
        for got, want in ((first[0], dx), (first[1], dw)):
            bar = 2 * ulp * want.abs().max().item() + 1e-6
            if not got.isfinite().all() or (got.float() - want).abs().max().item() > bar:
                raise RuntimeError("native source RMSNorm VJP differs from the FP32 closed form")


if StableQwen3RMSNorm is not None:

    class NativeSourceRMSNorm(StableQwen3RMSNorm):
        """A bf16 source norm whose forward and native-VJP trials passed on its
        device (grpo/rms_norm_native.py:98-101): the HIP forward and FP32 VJP
        of StableQwen3RMSNorm."""

    def use_compiled_source_rms_norm(model: torch.nn.Module) -> int:
        """Mark bf16 StableQwen3RMSNorm modules whose trials pass as
        NativeSourceRMSNorm, keeping every Parameter (grpo/rms_norm.py:44-84).
        Returns how many were swapped."""

        def ready(module) -> bool:
            if not isinstance(module, StableQwen3RMSNorm) or isinstance(module, NativeSourceRMSNorm):
                return False
            w = module.weight
            if w.dtype != torch.bfloat16 or not w.is_cuda:
                return False
            width = w.numel()
            return (kernel_runs(FORWARD_TRIAL, w, width,
                                lambda d, t, n: compiled_source_rms_trial(d, t, n, module.variance_epsilon))
                    and kernel_runs(NATIVE_VJP_TRIAL, w, width, native_source_rms_trial))

        return replace_norms(model, ready, lambda m: NativeSourceRMSNorm(m.weight.numel(), eps=m.variance_epsilon))
