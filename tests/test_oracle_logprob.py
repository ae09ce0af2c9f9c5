"""Pin the logprob oracle (CPU): closed forms, gradcheck, known answers."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import logprob as ref


def _inputs(n, d, v, seed=0, dtype=torch.float32, wscale=0.05):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g).to(dtype)
    w = (torch.randn(v, d, generator=g) * wscale).to(dtype)
    t = torch.randint(0, v, (n,), generator=g)
    return h, w, t


@pytest.mark.parametrize("chunk", [1, 7, 64, 4096])
def test_chunk_loop_matches_dense_closed_form(chunk):
    h, w, t = _inputs(129, 64, 501)
    lp, ent = ref.logprob_entropy_forward(h, w, t, chunk)
    want_lp, want_ent = ref.naive_logprob_entropy(h, w, t)
    torch.testing.assert_close(lp, want_lp, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ent, want_ent, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(ref.logprob_forward(h, w, t, chunk), want_lp, rtol=1e-5, atol=1e-6)


def test_hand_written_backward_matches_autograd_of_dense_form():
    h0, w0, t = _inputs(96, 48, 307, seed=1)
    g = torch.Generator().manual_seed(2)
    c_lp, c_ent = torch.randn(96, generator=g), torch.randn(96, generator=g)
    ha, wa = h0.clone().requires_grad_(), w0.clone().requires_grad_()
    lp, ent = ref.FusedLogprobEntropy.apply(ha, wa, t, 16)
    (c_lp * lp + c_ent * ent).sum().backward()
    hb, wb = h0.clone().requires_grad_(), w0.clone().requires_grad_()
    lp2, ent2 = ref.naive_logprob_entropy(hb, wb, t)
    (c_lp * lp2 + c_ent * ent2).sum().backward()
    torch.testing.assert_close(ha.grad, hb.grad, rtol=1e-4, atol=1e-6)
    torch.testing.assert_close(wa.grad, wb.grad, rtol=1e-4, atol=1e-6)
    # the logprob-only form equals the entropy form at g_ent = 0
    gh, gw = ref.logprob_backward(h0, w0, t, c_lp, 16, needs_weight_grad=True)
    _, ent0 = ref.logprob_entropy_forward(h0, w0, t, 16)
    gh2, gw2 = ref.logprob_entropy_backward(h0, w0, t, ent0, c_lp, torch.zeros(96), 16, True)
    torch.testing.assert_close(gh, gh2, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(gw, gw2, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("which", ["lp", "ent", "both"])
def test_gradcheck_fp64(which):
    h, w, t = _inputs(11, 6, 23, seed=3, dtype=torch.float64, wscale=0.1)
    h.requires_grad_()
    w.requires_grad_()

    def f(a, b):
        lp, ent = ref.FusedLogprobEntropy.apply(a, b, t, 4)
        return {"lp": lp, "ent": ent, "both": lp + 0.7 * ent}[which]

    assert torch.autograd.gradcheck(f, (h, w), eps=1e-6, atol=1e-8)


def test_entropy_within_analytic_bounds():
    h, w, t = _inputs(200, 32, 311, seed=4, wscale=0.2)
    _, ent = ref.logprob_entropy_forward(h * 3.0, w, t, 64)
    assert float(ent.min()) >= 0.0
    assert float(ent.max()) <= math.log(311) + 1e-5


@pytest.mark.parametrize("dtype,offset", [(torch.bfloat16, 256), (torch.float16, 2048)])
def test_known_answer_projection_precision(dtype, offset):
    # tests/test_accel_projection_precision.py:9-24 of the reference
    hidden = torch.tensor([[1, 1]], dtype=dtype)
    weight = torch.tensor([[offset, 1], [offset, 0]], dtype=dtype)
    target = torch.tensor([0])
    expected = torch.log_softmax(torch.nn.functional.linear(hidden.float(), weight.float()), -1)
    lp, ent = ref.logprob_entropy_forward(hidden, weight, target, 1)
    torch.testing.assert_close(lp, expected[:, 0], rtol=5e-4, atol=5e-4)
    torch.testing.assert_close(ent, -(expected.exp() * expected).sum(-1), rtol=5e-4, atol=5e-4)


@pytest.mark.parametrize("dtype,large", [(torch.bfloat16, 256), (torch.float16, 2048)])
def test_known_answer_weight_gradient(dtype, large):
    # tests/test_accel_projection_precision.py:27-41 of the reference
    hidden = torch.ones(3, 1, dtype=dtype)
    weight = torch.zeros(2, 1, dtype=dtype)
    target = torch.zeros(3, dtype=torch.long)
    coeff = torch.tensor([2 * large, 2, -2 * large], dtype=torch.float32)
    _, gw = ref.logprob_backward(hidden, weight, target, coeff, 1, needs_weight_grad=True)
    assert torch.equal(gw, torch.tensor([[1], [-1]], dtype=dtype))


def test_gathered_logprobs_rules():
    h, w, t = _inputs(8, 4, 17, seed=5)
    assert float(ref.gathered_logprobs(h, w, t, torch.ones(8, dtype=torch.bool))[0]) == 0.0
    out = ref.gathered_logprobs(h, w, t, torch.zeros(8, dtype=torch.bool))
    assert out.shape == (8,) and float(out.abs().sum()) == 0.0
