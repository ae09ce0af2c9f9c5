"""RMSNorm with the FP32 VJP, on the gfx950 kernels.

Drop-in for the reference's ``accel/rms_norm.py:7-70``: the forward keeps
the replaced ``Qwen3RMSNorm``'s primal operation order and both casts
(``w * T(float(x) * rstd)``) and saves ``(hidden, weight, rstd)``; the
backward is the FP32 VJP from that saved statistic, with ``dx`` cast to the
hidden dtype and ``dw`` to the weight dtype.  Both directions run in
``ts_rmsnorm_fwd`` / ``ts_rmsnorm_bwd`` (include/thundersync_hip.h); the
operator functions have no host path -- a CPU tensor raises.

The forward's bytes equal the stock module's on the GPU (the reference's
contract, "keep the original primal bytes", accel/rms_norm.py:46-52): the
kernel sums the squares in the order torch's reduction kernel uses for a
contiguous row and takes the correctly rounded rsqrt, as torch.rsqrt is.
That order is torch's, not this library's, so it is checked, not assumed:
the first forward of each (device, dtype, width, row class) -- the row class
is the only way the row count enters torch's reduction schedule -- computes
the primal both ways on the device and compares the bytes
(:func:`primal_matches_stock`).  On a mismatch ``THUNDERSYNC_HIP=require``
raises; ``auto`` takes the primal and its statistic from torch's own ops for
that class from then on, and the backward stays the HIP FP32 VJP.  A hidden
state whose rows are not contiguous takes torch's ops as well (torch reduces
a permuted tensor in another order).

``StableQwen3RMSNorm`` keeps the stock forward wherever the reference's does
or the kernels do not apply: CPU tensors, dtypes other than bf16/fp16, a
weight dtype that differs from the hidden dtype, shapes the kernels refuse
(``ts_rmsnorm_supported``), and a library that is switched off.  Elsewhere
it runs the HIP forward with and without grad alike, so a no-grad pass and
the recompute under grad give the same bytes.
"""

from __future__ import annotations

import threading

import torch

from . import _lib

try:  # the module swap targets transformers' Qwen3 norm when it is importable
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
except Exception:  # pragma: no cover - transformers absent
    Qwen3RMSNorm = None


def _check_device(hidden: torch.Tensor, weight: torch.Tensor) -> None:
    if not hidden.is_cuda or not weight.is_cuda:
        raise RuntimeError("thundersync_amd RMSNorm runs on the GPU only; got a CPU tensor")
    if hidden.dtype != weight.dtype:
        raise TypeError(
            f"hidden ({hidden.dtype}) and weight ({weight.dtype}) must share a dtype"
        )
    if weight.dim() != 1 or hidden.shape[-1] != weight.shape[0]:
        raise ValueError(
            f"weight {tuple(weight.shape)} does not match hidden {tuple(hidden.shape)}"
        )


def rms_norm_forward(hidden: torch.Tensor, weight: torch.Tensor, eps: float):
    """``(w * T(x * rstd), rstd)`` with ``rstd`` fp32 of shape ``[..., 1]``."""
    _check_device(hidden, weight)
    lib = _lib.require_library()
    x = hidden.contiguous()
    w = weight.contiguous()
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    y = torch.empty_like(x)
    rstd = torch.empty((*x.shape[:-1], 1), dtype=torch.float32, device=x.device)
    _lib.check(
        lib.ts_rmsnorm_fwd(
            x.data_ptr(), w.data_ptr(), y.data_ptr(), rstd.data_ptr(), rows, width,
            float(eps), _lib.dtype_code(x.dtype), _lib.stream_of(x),
        ),
        lambda: f"ts_rmsnorm_fwd(rows={rows}, width={width}, dtype={x.dtype})",
    )
    return y, rstd


_WORKSPACE_BYTES: dict[tuple[int, int], int] = {}


def _workspace_bytes(lib, rows: int, width: int) -> int:
    """ts_rmsnorm_bwd_workspace(rows, width), asked once per shape."""
    key = (rows, width)
    nbytes = _WORKSPACE_BYTES.get(key)
    if nbytes is None:
        if len(_WORKSPACE_BYTES) > 4096:
            _WORKSPACE_BYTES.clear()
        nbytes = _WORKSPACE_BYTES[key] = int(lib.ts_rmsnorm_bwd_workspace(rows, width))
    return nbytes


def rms_norm_backward(gradient, hidden, weight, rstd, needs=(True, True)):
    """``(dx, dw)`` of the FP32 VJP; either may be None when not needed."""
    _check_device(hidden, weight)
    lib = _lib.require_library()
    x = hidden.contiguous()
    w = weight.contiguous()
    dy = gradient.to(x.dtype).contiguous()
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    rs = rstd.contiguous().to(torch.float32)
    dx = torch.empty_like(x) if needs[0] else None
    dw = torch.empty_like(w) if needs[1] else None
    if dx is None and dw is None:
        return None, None
    ws_bytes = _workspace_bytes(lib, rows, width) if dw is not None else 0
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=x.device)
    _lib.check(
        lib.ts_rmsnorm_bwd(
            dy.data_ptr(), x.data_ptr(), w.data_ptr(), rs.data_ptr(),
            _lib.ptr(dx), _lib.ptr(dw), workspace.data_ptr(), ws_bytes, rows, width,
            _lib.dtype_code(x.dtype), _lib.stream_of(x),
        ),
        lambda: f"ts_rmsnorm_bwd(rows={rows}, width={width}, dtype={x.dtype})",
    )
    return dx, dw


def stock_forward(hidden: torch.Tensor, weight: torch.Tensor, eps: float):
    """``(primal, rstd)`` from torch's own ops, in the replaced module's order
    (accel/rms_norm.py:11-15): the bytes the HIP forward must reproduce."""
    x = hidden.to(torch.float32)
    rstd = torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return weight * (x * rstd).to(hidden.dtype), rstd


def _row_class(rows: int) -> int:
    """torch's reduction reads the row count only as min(2^floor(log2 rows), 512)."""
    c = 1
    while c * 2 <= min(rows, 512):
        c *= 2
    return c


_MATCHES: dict[tuple, bool] = {}
_MATCHES_LOCK = threading.Lock()


def primal_matches_stock(hidden: torch.Tensor, weight: torch.Tensor, eps: float) -> bool:
    """Whether ``ts_rmsnorm_fwd`` reproduces torch's primal and rstd bytes for
    this (device, dtype, width, row class); decided by one comparison on the
    first such call and cached.  Raises on a mismatch under
    ``THUNDERSYNC_HIP=require``."""
    width = hidden.shape[-1]
    rows = hidden.numel() // width if width else 0
    key = (hidden.device, hidden.dtype, width, _row_class(rows), float(eps))
    known = _MATCHES.get(key)
    if known is not None:
        return known
    with _MATCHES_LOCK:
        known = _MATCHES.get(key)
        if known is None:
            with torch.no_grad():
                y, rstd = rms_norm_forward(hidden, weight, eps)
                want_y, want_rstd = stock_forward(hidden, weight, eps)
            known = bool(torch.equal(y, want_y) and torch.equal(rstd, want_rstd))
            if not known and _lib.resolved_setting() == "require":
                raise RuntimeError(
                    f"ts_rmsnorm_fwd differs from torch's RMSNorm bytes for width {width}, "
                    f"{rows} rows, {hidden.dtype} (the installed torch reduces in another order)"
                )
            _MATCHES[key] = known
    return known


def reset_primal_checks() -> None:
    """Forget every byte comparison; the next forward per class checks again."""
    with _MATCHES_LOCK:
        _MATCHES.clear()


def primal_forward(hidden: torch.Tensor, weight: torch.Tensor, eps: float):
    """``(primal, rstd)`` with the stock module's bytes: the HIP forward where
    it has been shown to reproduce them, torch's ops otherwise."""
    if hidden.is_contiguous() and primal_matches_stock(hidden, weight, eps):
        return rms_norm_forward(hidden, weight, eps)
    _check_device(hidden, weight)
    return stock_forward(hidden, weight, eps)


class FP32RMSNormVJP(torch.autograd.Function):
    """``FP32RMSNormVJP.apply(hidden, weight, eps)`` as in accel/rms_norm.py:7-43."""

    @staticmethod
    def forward(ctx, hidden, weight, eps):
        primal, rstd = primal_forward(hidden, weight, eps)
        ctx.save_for_backward(hidden, weight, rstd)
        ctx.eps = eps
        return primal

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, gradient):
        hidden, weight, rstd = ctx.saved_tensors
        need = ctx.needs_input_grad
        dx, dw = rms_norm_backward(gradient, hidden, weight, rstd, (need[0], need[1]))
        return dx, dw, None


def hip_takes(hidden: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether the swapped module runs this call on the HIP kernels: bf16 or
    fp16 GPU tensors of one dtype, a shape both kernels take, and a library
    that is loaded (``THUNDERSYNC_HIP=require`` without one raises)."""
    if not (hidden.is_cuda and weight.is_cuda):
        return False
    if hidden.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != hidden.dtype:
        return False
    width = hidden.shape[-1] if hidden.dim() else 0
    if weight.dim() != 1 or width != weight.shape[0] or width == 0:
        return False
    lib = _lib.library()
    if lib is None:
        return False
    rows = hidden.numel() // width
    return bool(lib.ts_rmsnorm_supported(rows, width, _lib.stream_of(hidden)))


if Qwen3RMSNorm is not None:

    class StableQwen3RMSNorm(Qwen3RMSNorm):
        """Qwen3RMSNorm on the HIP kernels, primal bytes unchanged (accel/rms_norm.py:46-52).

        Under grad the forward is FP32RMSNormVJP (the FP32 VJP from the saved
        rstd); without grad it is the same forward with nothing saved.  Calls
        the kernels do not serve (:func:`hip_takes`) run the stock forward, as
        the reference's module does outside bf16/fp16 training.
        """

        def forward(self, hidden):
            if not hip_takes(hidden, self.weight):
                return super().forward(hidden)
            if torch.is_grad_enabled() and (hidden.requires_grad or self.weight.requires_grad):
                return FP32RMSNormVJP.apply(hidden, self.weight, self.variance_epsilon)
            return primal_forward(hidden, self.weight, self.variance_epsilon)[0]

    def replace_norms(model: torch.nn.Module, select, make) -> int:
        """Replace every named submodule ``m`` with ``select(m)`` true by
        ``make(m)``, a module built on the meta device that then takes ``m``'s
        own weight Parameter and training flag (no weight copy: optimizers
        and state dicts keep the original Parameter).  Returns the count."""
        count = 0
        for name, module in list(model.named_modules()):
            if not name or not select(module):
                continue
            with torch.device("meta"):
                replacement = make(module)
            replacement.weight = module.weight
            replacement.train(module.training)
            model.set_submodule(name, replacement)
            count += 1
        return count

    def use_stable_qwen3_rms_norm(model: torch.nn.Module) -> int:
        """Swap every Qwen3RMSNorm for StableQwen3RMSNorm (accel/rms_norm.py:55-70)."""
        return replace_norms(
            model,
            lambda m: isinstance(m, Qwen3RMSNorm) and not isinstance(m, StableQwen3RMSNorm),
            lambda m: StableQwen3RMSNorm(m.weight.numel(), eps=m.variance_epsilon),
        )
