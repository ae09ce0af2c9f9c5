"""Reduction of consumer adjoints at a forest boundary, on the gfx950 kernels.

Mirrors engine/boundary_adjoint.py of the reference: a shared segment has
several consumers, reverse mode produces one adjoint per consumer, and the
segment's backward needs ``existing + sum(consumer adjoints)``.  The
reference's fused custom kernel (``_triton_reduce``, :201-225) reads up to 16
consumer buffers in one launch and accumulates in fp32 before one cast to the
input dtype; ``reduce_boundary_adjoints(..., backend="hip")`` is that
reduction on ``ts_adjoint_reduce``, with the reference's input checks and
``None`` conventions (:123-153, :228-258).  Inputs that require grad take a
differentiable wrapper around the same kernel whose backward hands the
upstream derivative to every active adjoint and to ``existing``, the
derivative the reference's differentiable path defines (:156-171).

:func:`ledger_accumulate` is engine/streaming.py:2647-2665 (the FP32 adjoint
ledger) on ``ts_ledger_add``.

There is no CPU or eager path in this module: CPU tensors, fp64 and more than
:data:`HIP_MAX_DEGREE` adjoints per call raise (the reference's scheduler
flushes a partial reduction at that degree).
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence

import torch

from . import _lib

HIP_MAX_DEGREE = 16
SUPPORTED_BACKENDS = frozenset(("hip",))
_DTYPES = frozenset((torch.float16, torch.bfloat16, torch.float32))


def hip_boundary_adjoint_available() -> bool:
    """Whether this process can run the HIP reduction (library loaded, GPU visible)."""
    return torch.cuda.is_available() and _lib.library() is not None


def _validate_inputs(adjoints: Sequence[torch.Tensor | None], existing: torch.Tensor | None) -> list[torch.Tensor]:
    """boundary_adjoint.py:123-153: same-shape, same-dtype, same-device floats."""
    active = [a for a in adjoints if a is not None]
    reference = active[0] if active else existing
    if reference is None:
        return active
    if not reference.is_floating_point():
        raise TypeError(f"boundary adjoints must be floating-point tensors, got {reference.dtype}")
    for name, tensor in [*(("adjoint", a) for a in active), *((("existing", existing),) if existing is not None else ())]:
        if tensor.shape != reference.shape:
            raise ValueError(f"{name} shape {tuple(tensor.shape)} does not match {tuple(reference.shape)}")
        if tensor.dtype != reference.dtype:
            raise ValueError(f"{name} dtype {tensor.dtype} does not match {reference.dtype}")
        if tensor.device != reference.device:
            raise ValueError(f"{name} device {tensor.device} does not match {reference.device}")
    return active


def _kernel_ready(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (a copy only when it is neither)."""
    t = t.detach()
    if not t.is_contiguous() or t.data_ptr() % 16:
        t = t.clone(memory_format=torch.contiguous_format)
    return t


def _hip_reduce(active: Sequence[torch.Tensor], existing: torch.Tensor | None) -> torch.Tensor:
    reference = active[0] if active else existing
    if not reference.is_cuda:
        raise RuntimeError("thundersync_amd boundary-adjoint reduction runs on the GPU only; got a CPU tensor")
    if reference.dtype not in _DTYPES:
        raise TypeError(f"the HIP reduction takes float16, bfloat16 or float32, got {reference.dtype}")
    if len(active) > HIP_MAX_DEGREE:
        raise ValueError(f"at most {HIP_MAX_DEGREE} adjoints per reduction, got {len(active)}; "
                         "flush a partial reduction first")
    lib = _lib.require_library()
    if reference.numel() == 0:
        return torch.empty(reference.shape, dtype=reference.dtype, device=reference.device)
    ins = [_kernel_ready(a) for a in active]
    ex = _kernel_ready(existing) if existing is not None else None
    out = torch.empty(reference.shape, dtype=reference.dtype, device=reference.device)
    table = (ctypes.c_void_p * max(1, len(ins)))(*[t.data_ptr() for t in ins])
    _lib.check(
        lib.ts_adjoint_reduce(table, len(ins), ex.data_ptr() if ex is not None else None, out.data_ptr(),
                              out.numel(), _lib.dtype_code(out.dtype), _lib.stream_of(out)),
        f"ts_adjoint_reduce(degree={len(ins)}, n={out.numel()}, existing={ex is not None})",
    )
    return out


class _DifferentiableReduce(torch.autograd.Function):
    """The HIP reduction with d(out)/d(input) = identity for every input."""

    @staticmethod
    def forward(ctx, has_existing: bool, *tensors):
        existing = tensors[0] if has_existing else None
        return _hip_reduce(list(tensors[1:] if has_existing else tensors), existing)

    @staticmethod
    def backward(ctx, grad):
        n = len(ctx.needs_input_grad) - 1
        return (None, *[grad if ctx.needs_input_grad[1 + i] else None for i in range(n)])


def reduce_boundary_adjoints(adjoints: Sequence[torch.Tensor | None], *, existing: torch.Tensor | None = None,
                             backend: str = "hip") -> torch.Tensor | None:
    """Reduce consumer adjoints and optionally accumulate a parent adjoint
    (boundary_adjoint.py:228-258).

    ``None`` entries are ignored; with every entry and ``existing`` ``None``
    the result is ``None``.  Inputs are not modified; the result is a new
    tensor: ``cast(existing + sum(adjoints))`` with the sum in fp32 in input
    order (existing first).
    """
    if backend not in SUPPORTED_BACKENDS:
        raise ValueError(f"boundary adjoint backend must be one of {sorted(SUPPORTED_BACKENDS)}, got {backend!r}")
    active = _validate_inputs(adjoints, existing)
    if not active and existing is None:
        return None
    if any(t.requires_grad for t in active) or (existing is not None and existing.requires_grad):
        tensors = ([existing] if existing is not None else []) + active
        return _DifferentiableReduce.apply(existing is not None, *tensors)
    return _hip_reduce(active, existing)


def ledger_accumulate(ledgers: list[torch.Tensor | None], index: int, contribution: torch.Tensor) -> None:
    """Add one adjoint contribution to its owned FP32 ledger (streaming.py:2647-2665).

    The first contribution becomes the ledger as one widening copy; later ones
    are added after exact widening, so the ledger holds the same bits as
    widening every contribution and adding in order.
    """
    if not contribution.is_cuda:
        raise RuntimeError("thundersync_amd ledger accumulation runs on the GPU only; got a CPU tensor")
    if contribution.dtype not in _DTYPES:
        raise TypeError(f"the HIP ledger takes float16, bfloat16 or float32 contributions, got {contribution.dtype}")
    lib = _lib.require_library()
    c = _kernel_ready(contribution)
    ledger = ledgers[index]
    init = ledger is None
    if init:
        ledger = torch.empty(c.shape, dtype=torch.float32, device=c.device)
        ledgers[index] = ledger
    elif ledger.shape != c.shape or ledger.dtype != torch.float32 or not ledger.is_contiguous() or ledger.data_ptr() % 16:
        raise ValueError(f"ledger {tuple(ledger.shape)} {ledger.dtype} does not take a {tuple(c.shape)} contribution "
                         "(a contiguous 16-byte aligned fp32 tensor of the same shape)")
    _lib.check(
        lib.ts_ledger_add(ledger.data_ptr(), c.data_ptr(), c.numel(), _lib.dtype_code(c.dtype), int(init),
                          _lib.stream_of(c)),
        f"ts_ledger_add(n={c.numel()}, init={init})",
    )
