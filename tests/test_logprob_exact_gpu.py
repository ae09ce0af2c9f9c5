"""The fused logprob / entropy at fp32 and fp64 (the input-precision kernels).

The reference keeps FP32/FP64 inputs at their precision
(accel/fused_logprob.py:27-58) and holds them to its dense path in its own
accelerator tests: values at rtol 1e-5 / atol 1e-6 for chunks 1, 7, 64 and
4096 and gradients at rtol 1e-4 / atol 1e-6 in fp32
(tests/test_accel.py:33-65, tests/test_accel_entropy.py:39-101), and
fp64 gradcheck of the hand-written backward for the logprob, the entropy and
both together (tests/test_accel.py:68-77, tests/test_accel_entropy.py:
104-141).  The same checks here, at the same shapes and bars, against a
dense log-softmax on the host in the same dtype, and the C1 head shape
(hidden 128, vocabulary 1024) against the oracle's chunk loop.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import logprob as ref
from thundersync_amd import fused_logprob as fl

pytestmark = pytest.mark.gpu


def naive(hidden, weight, target):
    """Dense [N, V] log-softmax on the host in the inputs' dtype."""
    logits = hidden.cpu() @ weight.cpu().t()
    logp = torch.log_softmax(logits, dim=-1)
    lp = logp.gather(-1, target.cpu().unsqueeze(-1)).squeeze(-1)
    ent = -(logp.exp() * logp).sum(-1)
    return lp, ent


@pytest.mark.parametrize("chunk", [1, 7, 64, 4096])
def test_fp32_values_match_dense(cuda, chunk):
    print(f"fp32 gathered logprobs chunk={chunk}", flush=True)
    g = torch.Generator().manual_seed(chunk)
    n, d, v = 129, 64, 501
    h = torch.randn(n, d, generator=g)
    w = torch.randn(v, d, generator=g) * 0.05
    ids = torch.randint(0, v, (n,), generator=g)
    mask = torch.rand(n, generator=g) < 0.3
    got = fl.gathered_logprobs(h.to(cuda), w.to(cuda), ids.to(cuda), mask.to(cuda), chunk=chunk)
    assert got.dtype == torch.float32
    idx = mask.nonzero(as_tuple=True)[0]
    idx = idx[idx > 0]
    want = torch.zeros(n)
    want[idx] = naive(h[idx - 1], w, ids[idx])[0]
    torch.testing.assert_close(got.cpu(), want, rtol=1e-5, atol=1e-6)
    lp, ent = fl.fused_logprob_entropy(h.to(cuda), w.to(cuda), ids.to(cuda), chunk=chunk)
    want_lp, want_ent = naive(h, w, ids)
    torch.testing.assert_close(lp.cpu(), want_lp, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ent.cpu(), want_ent, rtol=1e-5, atol=1e-6)


def test_fp32_gradients_match_dense(cuda):
    """Both outputs read with independent coefficients; gradients to hidden
    and weight."""
    print("fp32 gradients, logprob and entropy", flush=True)
    g = torch.Generator().manual_seed(3)
    n, d, v = 96, 48, 307
    t = torch.randint(0, v, (n,), generator=g)
    c_lp, c_ent = torch.randn(n, generator=g), torch.randn(n, generator=g)
    h0 = torch.randn(n, d, generator=g)
    w0 = torch.randn(v, d, generator=g) * 0.05
    for with_entropy in (False, True):
        ha = h0.to(cuda).requires_grad_(True)
        wa = w0.to(cuda).requires_grad_(True)
        hb = h0.clone().requires_grad_(True)
        wb = w0.clone().requires_grad_(True)
        if with_entropy:
            lp, ent = fl.fused_logprob_entropy(ha, wa, t.to(cuda), chunk=16)
            (c_lp.to(cuda) * lp + c_ent.to(cuda) * ent).sum().backward()
            lp2, ent2 = naive(hb, wb, t)
            (c_lp * lp2 + c_ent * ent2).sum().backward()
        else:
            (c_lp.to(cuda) * fl.fused_logprob(ha, wa, t.to(cuda), chunk=16)).sum().backward()
            (c_lp * naive(hb, wb, t)[0]).sum().backward()
        torch.testing.assert_close(ha.grad.cpu(), hb.grad, rtol=1e-4, atol=1e-6)
        torch.testing.assert_close(wa.grad.cpu(), wb.grad, rtol=1e-4, atol=1e-6)


def _gradcheck_inputs(cuda, seed):
    g = torch.Generator().manual_seed(seed)
    n, d, v = 11, 6, 23
    h = torch.randn(n, d, generator=g, dtype=torch.float64).to(cuda).requires_grad_(True)
    w = (torch.randn(v, d, generator=g, dtype=torch.float64) * 0.1).to(cuda).requires_grad_(True)
    t = torch.randint(0, v, (n,), generator=g).to(cuda)
    return h, w, t


@pytest.mark.parametrize("which", ["logprob", "logprob_of_pair", "entropy", "both"])
def test_fp64_gradcheck(cuda, which):
    """The hand-written backward at fp64 against finite differences of the
    forward (eps 1e-6, atol 1e-8, as the reference's own gradchecks)."""
    print(f"fp64 gradcheck: {which}", flush=True)
    h, w, t = _gradcheck_inputs(cuda, 11)
    fns = {
        "logprob": lambda a, b: fl.fused_logprob(a, b, t, chunk=4),
        "logprob_of_pair": lambda a, b: fl.fused_logprob_entropy(a, b, t, chunk=4)[0],
        "entropy": lambda a, b: fl.fused_logprob_entropy(a, b, t, chunk=4)[1],
        "both": lambda a, b: (lambda lp, ent: lp + 0.7 * ent)(*fl.fused_logprob_entropy(a, b, t, chunk=4)),
    }
    assert torch.autograd.gradcheck(fns[which], (h, w), eps=1e-6, atol=1e-8)


def test_fp64_outputs_keep_their_precision(cuda):
    print("fp64 values against the host in fp64", flush=True)
    g = torch.Generator().manual_seed(5)
    n, d, v = 40, 24, 333
    h = torch.randn(n, d, generator=g, dtype=torch.float64)
    w = torch.randn(v, d, generator=g, dtype=torch.float64) * 0.3
    t = torch.randint(0, v, (n,), generator=g)
    lp, ent = fl.fused_logprob_entropy(h.to(cuda), w.to(cuda), t.to(cuda), chunk=8)
    assert lp.dtype == torch.float64 and ent.dtype == torch.float64
    want_lp, want_ent = naive(h, w, t)
    torch.testing.assert_close(lp.cpu(), want_lp, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ent.cpu(), want_ent, rtol=1e-12, atol=1e-12)


def test_fp32_entropy_within_its_bounds_and_frozen_weight(cuda):
    """0 <= H <= log V on sharpened rows; a frozen head gets no gradient."""
    print("fp32 entropy bounds, frozen head", flush=True)
    g = torch.Generator().manual_seed(7)
    n, d, v = 200, 32, 311
    h = (torch.randn(n, d, generator=g) * 3.0).to(cuda).requires_grad_(True)
    w = (torch.randn(v, d, generator=g) * 0.2).to(cuda)
    t = torch.randint(0, v, (n,), generator=g).to(cuda)
    lp, ent = fl.fused_logprob_entropy(h, w, t, chunk=64)
    assert float(ent.min()) >= 0.0 and float(ent.max()) <= math.log(v) + 1e-5
    (lp.sum() + ent.sum()).backward()
    assert h.grad is not None and w.grad is None


def test_fp32_c1_head_against_the_oracle_chunk_loop(cuda):
    """C1's head (hidden 128, vocabulary 1024, fp32) through the entropy
    operator and its backward with a trainable head, against the oracle's
    restatement of the reference's chunk loop run on the host in fp32."""
    print("fp32 C1 head: 150 rows, hidden 128, vocab 1024", flush=True)
    g = torch.Generator().manual_seed(1)
    n, d, v = 150, 128, 1024
    h = torch.randn(n, d, generator=g)
    w = torch.randn(v, d, generator=g) * 0.02
    t = torch.randint(0, v, (n,), generator=g)
    g_lp, g_ent = torch.randn(n, generator=g), torch.randn(n, generator=g)
    hd, wd = h.to(cuda).requires_grad_(True), w.to(cuda).requires_grad_(True)
    lp, ent = fl.fused_logprob_entropy(hd, wd, t.to(cuda), chunk=64)
    (lp * g_lp.to(cuda) + ent * g_ent.to(cuda)).sum().backward()
    want_lp, want_ent = ref.logprob_entropy_forward(h, w, t, chunk=64)
    want_gh, want_gw = ref.logprob_entropy_backward(h, w, t, want_ent, g_lp, g_ent, chunk=64,
                                                    needs_weight_grad=True)
    torch.testing.assert_close(lp.detach().cpu(), want_lp, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(ent.detach().cpu(), want_ent, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(hd.grad.cpu(), want_gh, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(wd.grad.cpu(), want_gw, rtol=1e-4, atol=1e-6)


def test_fp32_strided_head_view_and_ragged_edges(cuda):
    """A head that is a column slice of a wider tensor (row stride above the
    hidden dim), rows, dim and vocabulary off the 64-wide tiles; against the
    host in fp64."""
    print("fp32 strided head: 301 rows, dim 77, vocab 5003", flush=True)
    g = torch.Generator().manual_seed(9)
    n, d, v = 301, 77, 5003
    h = torch.randn(n, d, generator=g)
    wide = torch.randn(v, d + 13, generator=g) * 0.1
    t = torch.randint(0, v, (n,), generator=g)
    wd = wide.to(cuda)[:, :d].requires_grad_(False)
    hd = h.to(cuda).requires_grad_(True)
    lp = fl.fused_logprob(hd, wd, t.to(cuda), chunk=128)
    lp.sum().backward()
    hx = h.double().requires_grad_(True)
    want = naive(hx, wide[:, :d].double(), t)[0]
    want.sum().backward()
    torch.testing.assert_close(lp.detach().cpu().double(), want.detach(), rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(hd.grad.cpu().double(), hx.grad, rtol=1e-4, atol=1e-5)
