"""CPU restatement of the reference's boundary-adjoint reduction and FP32
ledger -- TEST INFRASTRUCTURE ONLY (the parity tests' checker and bench.py's
CPU baseline; the product never imports it).

* :func:`reduce_sequential` -- engine/boundary_adjoint.py:156-180, the
  PyTorch reference path: ``existing.clone()`` (or zeros) and one in-place
  ``add_`` per adjoint, rounding to the input dtype after every addition.
* :func:`reduce_fp32` -- the fused custom kernel's declared semantics
  (engine/boundary_adjoint.py:75-115: fp32 accumulator starting from the
  existing adjoint or zeros, adjoints added in order, one cast at the store),
  which is also the oracle the reference's own test builds for that kernel
  (tests/test_boundary_adjoint.py:120-131).
* :func:`ledger_accumulate` -- engine/streaming.py:2647-2665: the first
  contribution widened into an FP32 (FP64 for FP64 input) ledger, later ones
  added by a mixed-dtype ``add_``.

Pinned in tests/test_oracle_boundary_adjoint.py by exact integer sums, by the
fp32 identity of the two reductions, and by the reference's own bf16 audit
(fp32 accumulation about 3x closer to the exact sum than sequential adds at
degree 16).
"""

from __future__ import annotations

from collections.abc import Sequence

import torch


def _active(adjoints: Sequence[torch.Tensor | None]) -> list[torch.Tensor]:
    return [a for a in adjoints if a is not None]


def reduce_sequential(adjoints: Sequence[torch.Tensor | None], existing: torch.Tensor | None = None):
    active = _active(adjoints)
    if existing is not None:
        result = existing.clone()
    elif active:
        result = torch.zeros_like(active[0])
    else:
        return None
    for a in active:
        result.add_(a)
    return result


def reduce_fp32(adjoints: Sequence[torch.Tensor | None], existing: torch.Tensor | None = None):
    active = _active(adjoints)
    reference = active[0] if active else existing
    if reference is None:
        return None
    total = existing.float() if existing is not None else torch.zeros(reference.shape, dtype=torch.float32)
    for a in active:
        total = total + a.float()
    return total.to(reference.dtype)


def ledger_accumulate(ledgers: list[torch.Tensor | None], index: int, contribution: torch.Tensor) -> None:
    accumulator = ledgers[index]
    if accumulator is None:
        dtype = torch.float64 if contribution.dtype == torch.float64 else torch.float32
        ledgers[index] = contribution.to(dtype=dtype, copy=True)
    else:
        accumulator.add_(contribution)
