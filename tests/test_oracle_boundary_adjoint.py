"""Pin the boundary-adjoint oracle (CPU).

* Integer-valued adjoints whose every partial sum is exactly representable:
  both reductions equal the exact sum, in every dtype.
* fp32 inputs: the fp32-accumulating reduction and the sequential one are the
  same additions in the same order, hence bit-identical.
* The reference's own bf16 audit (tests/test_boundary_adjoint.py:133-145):
  at degree 16 on N(0, 1) adjoints, fp32 accumulation is about 0.0016
  relative L2 from the exact sum and sequential bf16 adds about 0.005.
* The ledger: integer contributions give the exact sum; the first
  contribution is a widening copy (FP64 input keeps an FP64 ledger).
"""

from __future__ import annotations

import pytest
import torch

from oracle import boundary_adjoint as ob


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_exact_integer_sums(dtype):
    g = torch.Generator().manual_seed(3)
    adj = [torch.randint(-8, 9, (5, 7), generator=g).to(dtype) for _ in range(16)]
    existing = torch.randint(-8, 9, (5, 7), generator=g).to(dtype)
    exact = existing.double() + sum(a.double() for a in adj)
    for fn in (ob.reduce_fp32, ob.reduce_sequential):
        got = fn([None, *adj, None], existing)
        assert got.dtype == dtype
        assert torch.equal(got.double(), exact)
    assert torch.equal(ob.reduce_fp32(adj[:1]).double(), adj[0].double())
    assert ob.reduce_fp32([None]) is None and ob.reduce_sequential([None]) is None


def test_fp32_reductions_are_identical():
    g = torch.Generator().manual_seed(4)
    adj = [torch.randn(257, generator=g) for _ in range(9)]
    existing = torch.randn(257, generator=g)
    assert torch.equal(ob.reduce_fp32(adj, existing), ob.reduce_sequential(adj, existing))


@pytest.mark.parametrize("shape", [(257,), (7, 513), (2, 3, 65)])
def test_reference_bf16_audit(shape):
    g = torch.Generator().manual_seed(2016)
    adj = [torch.randn(shape, generator=g).to(torch.bfloat16) for _ in range(16)]
    existing = torch.randn(shape, generator=g).to(torch.bfloat16)
    exact = existing.double() + sum(a.double() for a in adj)
    scale = exact.norm()
    fused = (ob.reduce_fp32(adj, existing).double() - exact).norm() / scale
    seq = (ob.reduce_sequential(adj, existing).double() - exact).norm() / scale
    assert 0.0005 < fused < 0.003 and 0.003 < seq < 0.009 and fused < seq / 2, (fused, seq)


def test_ledger():
    g = torch.Generator().manual_seed(5)
    parts = [torch.randint(-100, 101, (33,), generator=g).to(torch.bfloat16) for _ in range(5)]
    ledgers = [None, None]
    for p in parts:
        ob.ledger_accumulate(ledgers, 1, p)
    assert ledgers[0] is None and ledgers[1].dtype == torch.float32
    assert torch.equal(ledgers[1].double(), sum(p.double() for p in parts))
    first = parts[0]
    led = [None]
    ob.ledger_accumulate(led, 0, first)
    assert led[0].data_ptr() != first.data_ptr() and torch.equal(led[0], first.float())
    led64 = [None]
    ob.ledger_accumulate(led64, 0, torch.ones(3, dtype=torch.float64))
    assert led64[0].dtype == torch.float64
