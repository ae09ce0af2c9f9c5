"""HIP boundary-adjoint reduction and FP32 ledger against the CPU oracle.

Bar: bit-exact.  The kernel adds in fp32 in input order (existing first) and
casts once, which is what ``oracle.boundary_adjoint.reduce_fp32`` computes;
fp32 addition is correctly rounded, so the same additions in the same order
give the same bits.  The test grid is the reference's own
(tests/test_boundary_adjoint.py: degrees 1, 2, 5, 16; its CPU and CUDA
shapes; fp16, bf16, fp32; missing adjoints; an existing parent adjoint), plus
sizes that are not multiples of the kernel's eight-element vectors,
non-contiguous and misaligned inputs, the full bench size, and the
reference's edge cases (all adjoints missing, mismatched inputs, higher-order
semantics).
"""

from __future__ import annotations

import pytest
import torch

from oracle import boundary_adjoint as ob
from thundersync_amd import boundary_adjoint as hip

pytestmark = pytest.mark.gpu

SHAPES = [(17,), (3, 11), (2, 3, 7), (257,), (7, 513), (2, 3, 65), (8,), (4096,)]


@pytest.mark.parametrize("degree", [1, 2, 5, 16])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("with_existing", [True, False])
def test_matches_fp32_oracle_bitwise(cuda, degree, shape, dtype, with_existing):
    g = torch.Generator().manual_seed(1000 + degree)
    adj = [torch.randn(shape, generator=g).to(dtype) for _ in range(degree)]
    existing = torch.randn(shape, generator=g).to(dtype) if with_existing else None
    inputs = [None, *adj, None]
    want = ob.reduce_fp32(inputs, existing)
    dev_in = [None if a is None else a.to(cuda) for a in inputs]
    dev_ex = existing.to(cuda) if existing is not None else None
    before = [a.clone() for a in dev_in if a is not None]
    got = hip.reduce_boundary_adjoints(dev_in, existing=dev_ex)
    torch.cuda.synchronize()
    assert got.dtype == dtype and got.shape == torch.Size(shape)
    assert torch.equal(got.cpu(), want)
    assert all(torch.equal(a, b) for a, b in zip([a for a in dev_in if a is not None], before))
    if dev_ex is not None:
        assert got.data_ptr() != dev_ex.data_ptr()


def test_bf16_beats_sequential_adds_as_the_reference_audit_states(cuda):
    g = torch.Generator().manual_seed(2016)
    adj = [torch.randn(7, 513, generator=g).to(torch.bfloat16) for _ in range(16)]
    existing = torch.randn(7, 513, generator=g).to(torch.bfloat16)
    exact = existing.double() + sum(a.double() for a in adj)
    got = hip.reduce_boundary_adjoints([a.to(cuda) for a in adj], existing=existing.to(cuda)).cpu()
    seq = ob.reduce_sequential(adj, existing)
    err = lambda x: float((x.double() - exact).norm() / exact.norm())
    assert err(got) < err(seq) / 2, (err(got), err(seq))


def test_zero_missing_and_existing_only(cuda):
    base = torch.arange(12, dtype=torch.float32, device=cuda).reshape(3, 4)
    got = hip.reduce_boundary_adjoints([None, torch.zeros_like(base), base, None])
    assert torch.equal(got, base)
    existing = torch.randn(9, device=cuda)
    got = hip.reduce_boundary_adjoints([None, None], existing=existing)
    assert torch.equal(got, existing) and got.data_ptr() != existing.data_ptr()
    assert hip.reduce_boundary_adjoints([None, None]) is None
    empty = torch.zeros(0, 5, dtype=torch.bfloat16, device=cuda)
    assert hip.reduce_boundary_adjoints([empty, empty]).shape == (0, 5)


def test_non_contiguous_and_misaligned_inputs(cuda):
    g = torch.Generator().manual_seed(9)
    big = torch.randn(4, 301, generator=g).to(torch.bfloat16).to(cuda)
    a = big[:, 1:300]            # non-contiguous
    b = big.flatten()[3:3 + 4 * 299].view(4, 299)  # contiguous, 6 bytes past a 16-byte boundary
    want = ob.reduce_fp32([a.cpu(), b.cpu()], None)
    got = hip.reduce_boundary_adjoints([a, b])
    assert torch.equal(got.cpu(), want) and got.is_contiguous()


def test_full_bench_size(cuda):
    g = torch.Generator(device=cuda).manual_seed(0)
    adj = [torch.randn(4096, 4096, generator=g, device=cuda, dtype=torch.bfloat16) for _ in range(16)]
    existing = torch.randn(4096, 4096, generator=g, device=cuda, dtype=torch.bfloat16)
    got = hip.reduce_boundary_adjoints(adj, existing=existing)
    want = ob.reduce_fp32([a.cpu() for a in adj], existing.cpu())
    assert torch.equal(got.cpu(), want)


def test_input_errors(cuda):
    with pytest.raises(ValueError, match="shape"):
        hip.reduce_boundary_adjoints([torch.zeros(2, device=cuda), torch.zeros(3, device=cuda)])
    with pytest.raises(ValueError, match="dtype"):
        hip.reduce_boundary_adjoints([torch.zeros(2, device=cuda)],
                                     existing=torch.zeros(2, dtype=torch.float64, device=cuda))
    with pytest.raises(ValueError, match="backend"):
        hip.reduce_boundary_adjoints([torch.zeros(2, device=cuda)], backend="cuda")
    with pytest.raises(TypeError, match="floating-point"):
        hip.reduce_boundary_adjoints([torch.zeros(2, dtype=torch.int32, device=cuda)])
    with pytest.raises(TypeError, match="float16, bfloat16 or float32"):
        hip.reduce_boundary_adjoints([torch.zeros(2, dtype=torch.float64, device=cuda)])
    with pytest.raises(ValueError, match="at most 16"):
        hip.reduce_boundary_adjoints([torch.zeros(2, device=cuda)] * 17)
    with pytest.raises(RuntimeError, match="GPU only"):
        hip.reduce_boundary_adjoints([torch.zeros(2)])


def test_higher_order_semantics(cuda):
    """The reference's test_higher_order_semantics_use_differentiable_reference."""
    a = torch.randn(7, device=cuda, requires_grad=True)
    b = torch.randn(7, device=cuda, requires_grad=True)
    existing = torch.randn(7, device=cuda, requires_grad=True)
    upstream = torch.linspace(-1.0, 1.0, 7, device=cuda)
    out = hip.reduce_boundary_adjoints([a, None, b], existing=existing)
    (out * upstream).sum().backward()
    for t in (a, b, existing):
        assert torch.equal(t.grad, upstream)
    c = torch.randn(7, device=cuda, requires_grad=True)
    hip.reduce_boundary_adjoints([c]).sum().backward()
    assert torch.equal(c.grad, torch.ones_like(c))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n", [1, 8, 37, 4099])
def test_ledger_matches_oracle(cuda, dtype, n):
    g = torch.Generator().manual_seed(n)
    parts = [torch.randn(n, generator=g).to(dtype) for _ in range(4)]
    want = [None]
    for p in parts:
        ob.ledger_accumulate(want, 0, p)
    got = [None]
    for p in parts:
        hip.ledger_accumulate(got, 0, p.to(cuda))
    torch.cuda.synchronize()
    assert got[0].dtype == torch.float32 and torch.equal(got[0].cpu(), want[0])
    with pytest.raises(TypeError, match="contributions"):
        hip.ledger_accumulate([None], 0, torch.zeros(3, dtype=torch.float64, device=cuda))
