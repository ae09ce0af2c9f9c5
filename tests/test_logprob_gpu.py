"""HIP fused logprob / entropy against the CPU oracle (the reference's chunk loop).

Bars: per-token logprobs within 1e-3 (the north star's bar) and entropies
within 1e-3, on identical bf16 inputs; grad wrt hidden within 1e-2 x
max|ref| (both sides round dlogits to bf16 before the VJP GEMM, as the
reference does, and round the result to bf16).  The full-size C3 check
compares sampled rows: every row's outputs and gradient depend on that row
alone, so a sample is an exact parity check of those rows.
"""

from __future__ import annotations

import pytest
import torch

from oracle import logprob as ref
from thundersync_amd import fused_logprob as hip

pytestmark = pytest.mark.gpu


def _inputs(n, d, v, seed, wscale=0.02):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g).to(torch.bfloat16)
    w = (torch.randn(v, d, generator=g) * wscale).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g)
    g_lp = torch.randn(n, generator=g)
    g_ent = torch.randn(n, generator=g)
    return h, w, t, g_lp, g_ent


def rel_close(got, want, bar, what):
    got, want = got.detach().float().cpu(), want.detach().float().cpu()
    err = (got - want).abs().max().item()
    scale = max(want.abs().max().item(), 1e-6)
    assert err <= bar * scale, f"{what}: max-abs {err:.3g} > {bar} x {scale:.3g}"


SHAPES = [(129, 64, 501), (64, 32, 203), (1000, 256, 4099), (300, 4096, 32000), (5, 8, 8), (257, 128, 1024)]


@pytest.mark.parametrize("n,d,v", SHAPES)
def test_entropy_values_and_grad(cuda, n, d, v):
    print(f"logprob entropy n={n} d={d} v={v}", flush=True)
    h, w, t, g_lp, g_ent = _inputs(n, d, v, seed=n + d + v)
    want_lp, want_ent = ref.logprob_entropy_forward(h, w, t, 1024)
    want_gh, _ = ref.logprob_entropy_backward(h, w, t, want_ent, g_lp, g_ent, 1024)
    hc = h.to(cuda).requires_grad_()
    lp, ent = hip.fused_logprob_entropy(hc, w.to(cuda), t.to(cuda))
    assert lp.dtype == torch.float32 and ent.dtype == torch.float32
    (lp * g_lp.to(cuda) + ent * g_ent.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    torch.testing.assert_close(lp.cpu(), want_lp, rtol=0, atol=1e-3)
    torch.testing.assert_close(ent.cpu(), want_ent, rtol=0, atol=1e-3)
    rel_close(hc.grad, want_gh, 1e-2, "grad hidden")


@pytest.mark.parametrize("n,d,v", SHAPES[:4])
def test_logprob_only_values_and_grad(cuda, n, d, v):
    print(f"logprob n={n} d={d} v={v}", flush=True)
    h, w, t, g_lp, _ = _inputs(n, d, v, seed=2 * n + v)
    want = ref.logprob_forward(h, w, t, 1024)
    want_gh, _ = ref.logprob_backward(h, w, t, g_lp, 1024)
    hc = h.to(cuda).requires_grad_()
    lp = hip.fused_logprob(hc, w.to(cuda), t.to(cuda), chunk=7)
    (lp * g_lp.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    torch.testing.assert_close(lp.cpu(), want, rtol=0, atol=1e-3)
    rel_close(hc.grad, want_gh, 1e-2, "grad hidden")


def test_weight_gradient_and_frozen_weight(cuda):
    h, w, t, g_lp, g_ent = _inputs(96, 48, 307, seed=11, wscale=0.05)
    _, ent = ref.logprob_entropy_forward(h, w, t, 16)
    want_gh, want_gw = ref.logprob_entropy_backward(h, w, t, ent, g_lp, g_ent, 16, needs_weight_grad=True)
    hc, wc = h.to(cuda).requires_grad_(), w.to(cuda).requires_grad_()
    lp, en = hip.fused_logprob_entropy(hc, wc, t.to(cuda), chunk=16)
    (lp * g_lp.to(cuda) + en * g_ent.to(cuda)).sum().backward()
    rel_close(hc.grad, want_gh, 1e-2, "grad hidden")
    rel_close(wc.grad, want_gw, 1e-2, "grad weight")
    # frozen weight: no weight gradient is formed
    hc2 = h.to(cuda).requires_grad_()
    w2 = w.to(cuda)
    hip.fused_logprob(hc2, w2, t.to(cuda), chunk=8).sum().backward()
    assert hc2.grad is not None and w2.grad is None


def test_known_answer_precision_cases(cuda):
    # accel precision cases of the reference (tests/test_accel_projection_precision.py:9-41)
    hidden = torch.tensor([[1, 1]], dtype=torch.bfloat16, device=cuda)
    weight = torch.tensor([[256, 1], [256, 0]], dtype=torch.bfloat16, device=cuda)
    target = torch.tensor([0], device=cuda)
    expected = torch.log_softmax(torch.nn.functional.linear(hidden.float(), weight.float()), -1)
    lp, ent = hip.fused_logprob_entropy(hidden, weight, target, chunk=1)
    torch.testing.assert_close(lp, expected[:, 0], rtol=5e-4, atol=5e-4)
    torch.testing.assert_close(ent, -(expected.exp() * expected).sum(-1), rtol=5e-4, atol=5e-4)
    hidden = torch.ones(3, 1, dtype=torch.bfloat16, device=cuda)
    weight = torch.zeros(2, 1, dtype=torch.bfloat16, device=cuda, requires_grad=True)
    target = torch.zeros(3, dtype=torch.long, device=cuda)
    coeff = torch.tensor([512.0, 2.0, -512.0], device=cuda)
    (coeff * hip.fused_logprob(hidden, weight, target, chunk=1)).sum().backward()
    assert torch.equal(weight.grad, torch.tensor([[1], [-1]], dtype=torch.bfloat16, device=cuda))


def test_gathered_logprobs_and_edge_cases(cuda):
    h, w, t, _, _ = _inputs(64, 32, 203, seed=5)
    mask = torch.rand(64, generator=torch.Generator().manual_seed(1)) < 0.3
    got = hip.gathered_logprobs(h.to(cuda), w.to(cuda), t.to(cuda), mask.to(cuda), chunk=16)
    want = ref.gathered_logprobs(h, w, t, mask, 16)
    torch.testing.assert_close(got.cpu(), want, rtol=0, atol=1e-3)
    ones = torch.ones(64, dtype=torch.bool, device=cuda)
    assert float(hip.gathered_logprobs(h.to(cuda), w.to(cuda), t.to(cuda), ones)[0]) == 0.0
    zeros = torch.zeros(64, dtype=torch.bool, device=cuda)
    assert float(hip.gathered_logprobs(h.to(cuda), w.to(cuda), t.to(cuda), zeros).abs().sum()) == 0.0
    # empty input
    lp, ent = hip.fused_logprob_entropy(h[:0].to(cuda), w.to(cuda), t[:0].to(cuda))
    assert lp.shape == (0,) and ent.shape == (0,)
    # a target outside the vocabulary is reported as NaN, not a wrong number
    bad = t.clone()
    bad[3] = 203
    lp = hip.fused_logprob(h.to(cuda), w.to(cuda), bad.to(cuda))
    assert torch.isnan(lp[3]).item() and not torch.isnan(lp[:3]).any().item()


def test_out_of_range_targets_match_no_vocabulary_row(cuda):
    """A target outside [0, vocab) adds no one-hot term to dlogits, however large (no 32-bit wrap)."""
    g = torch.Generator().manual_seed(11)
    h = torch.randn(8, 32, generator=g).to(torch.bfloat16)
    w = (torch.randn(203, 32, generator=g) * 0.05).to(torch.bfloat16)
    t = torch.randint(0, 203, (8,), generator=g)
    grads = []
    for bad in (203, 2**32 + 5, -1):
        tt = t.clone()
        tt[2] = bad
        hc = h.to(cuda).requires_grad_()
        lp = hip.fused_logprob(hc, w.to(cuda), tt.to(cuda))
        lp.backward(torch.ones_like(lp))  # row 2 (NaN logprob) still has an upstream gradient
        grads.append(hc.grad.cpu())
    assert torch.equal(grads[0], grads[1]) and torch.equal(grads[0], grads[2])


def test_target_check_names_the_row(cuda, monkeypatch):
    h = torch.randn(6, 8, dtype=torch.bfloat16, device=cuda)
    w = torch.randn(16, 8, dtype=torch.bfloat16, device=cuda)
    t = torch.tensor([1, 2, 3, 16, 0, -1], device=cuda)
    monkeypatch.setenv(hip.CHECK_TARGETS_ENV, "1")
    with pytest.raises(ValueError, match=r"target\[3\] = 16 is outside the vocabulary \[0, 16\)"):
        hip.fused_logprob(h, w, t)
    monkeypatch.setenv(hip.CHECK_TARGETS_ENV, "0")
    assert torch.isnan(hip.fused_logprob(h, w, t)[3]).item()


def test_validation_errors(cuda):
    h = torch.randn(4, 8, dtype=torch.bfloat16, device=cuda)
    w = torch.randn(16, 8, dtype=torch.bfloat16, device=cuda)
    t = torch.zeros(4, dtype=torch.long, device=cuda)
    with pytest.raises(ValueError, match=r"hidden must be \[N, D\]"):
        hip.fused_logprob(h[0], w, t)
    with pytest.raises(ValueError, match="one entry per hidden row"):
        hip.fused_logprob(h, w, t[:3])
    with pytest.raises(ValueError, match="does not match hidden dim"):
        hip.fused_logprob(h, w[:, :4], t)
    with pytest.raises(TypeError):  # one dtype for hidden and head
        hip.fused_logprob(h.float(), w, t)
    with pytest.raises(TypeError):  # fp32 / fp64 run at their precision; integer tensors do not
        hip.fused_logprob(h.to(torch.int32), w.to(torch.int32), t)
    with pytest.raises(RuntimeError, match="GPU only"):
        hip.fused_logprob(h.cpu(), w.cpu(), t.cpu())


def test_c3_full_size_sampled_rows(cuda):
    """C3 shapes: 16384 x 4096 hidden, 151936 x 4096 head, 70% scored rows gated first."""
    n, d, v = 16384, 4096, 151936
    g = torch.Generator(device=cuda).manual_seed(0)
    h = torch.randn(n, d, generator=g, device=cuda, dtype=torch.bfloat16)
    w = (torch.randn(v, d, generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device=cuda)
    adv = torch.randn(n, generator=g, device=cuda)
    mask = torch.rand(n, generator=g, device=cuda) < 0.7
    idx = mask.nonzero(as_tuple=True)[0]
    hs = h.index_select(0, idx).requires_grad_()
    print(f"c3 full size: scored rows {idx.numel()}", flush=True)
    lp, ent = hip.fused_logprob_entropy(hs, w, t[idx])
    (lp * adv[idx]).sum().backward()
    torch.cuda.synchronize()
    sample = torch.arange(0, idx.numel(), max(1, idx.numel() // 24), device=cuda)[:24]
    sample = torch.cat([sample, torch.tensor([idx.numel() - 1], device=cuda)])
    hs_cpu = hs.detach()[sample].cpu()
    w_cpu = w.cpu()
    t_cpu = t[idx][sample].cpu()
    want_lp, want_ent = ref.logprob_entropy_forward(hs_cpu, w_cpu, t_cpu, 1024)
    want_gh, _ = ref.logprob_entropy_backward(hs_cpu, w_cpu, t_cpu, want_ent, adv[idx][sample].cpu(),
                                              torch.zeros(sample.numel()), 1024)
    torch.testing.assert_close(lp[sample].cpu(), want_lp, rtol=0, atol=1e-3)
    torch.testing.assert_close(ent[sample].cpu(), want_ent, rtol=0, atol=1e-3)
    rel_close(hs.grad[sample], want_gh, 1e-2, "grad hidden (sampled rows)")


def test_weight_gradient_c3_head(cuda):
    """The hand-written weight gradient at the C3 head's shape (151936 x 4096):
    two 128-row dlogits blocks accumulated in fp32 and cast once, against the
    oracle's needs_weight_grad path (fused_logprob.py:176-193), every row."""
    n, d, v = 256, 4096, 151936
    h, w, t, g_lp, g_ent = _inputs(n, d, v, seed=23)
    print(f"weight gradient n={n} d={d} v={v} chunk=128", flush=True)
    _, ent = ref.logprob_entropy_forward(h, w, t, 128)
    want_gh, want_gw = ref.logprob_entropy_backward(h, w, t, ent, g_lp, g_ent, 128, needs_weight_grad=True)
    hc, wc = h.to(cuda).requires_grad_(), w.to(cuda).requires_grad_()
    lp, en = hip.fused_logprob_entropy(hc, wc, t.to(cuda), chunk=128)
    (lp * g_lp.to(cuda) + en * g_ent.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    rel_close(hc.grad, want_gh, 1e-2, "grad hidden")
    rel_close(wc.grad, want_gw, 1e-2, "grad weight")
    # the target rows carry the one-hot term: check them on their own scale too
    rows = t.unique()
    rel_close(wc.grad[rows.to(cuda)], want_gw[rows], 1e-2, "grad weight (target rows)")


def test_backward_memory_is_one_chunk(cuda):
    """Peak extra device memory of the backward is one bf16 dlogits block of
    two chunks of rows -- the bytes of the reference's own fp32 [chunk, V]
    logit block (fused_logprob.py:137-175) -- plus the grad_hidden workspace:
    the reference's O(chunk * V) (fused_logprob.py:20-24), not O(N * V)."""
    from thundersync_amd import _lib

    n, d, v, chunk = 4096, 4096, 151936, 1024
    g = torch.Generator(device=cuda).manual_seed(3)
    h = torch.randn(n, d, generator=g, device=cuda, dtype=torch.bfloat16).requires_grad_()
    w = (torch.randn(v, d, generator=g, device=cuda) * 0.02).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g, device=cuda)
    lp, ent = hip.fused_logprob_entropy(h, w, t, chunk=chunk)
    upstream = torch.randn(n, generator=g, device=cuda)
    loss = (lp * upstream).sum()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(cuda)
    before = torch.cuda.memory_allocated(cuda)
    loss.backward()
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated(cuda) - before
    block = hip.backward_block_rows(n, chunk)
    dl_bytes = block * ((v + 7) // 8 * 8) * 2
    ws_bytes = int(_lib.require_library().ts_logprob_grad_hidden_workspace(block, d, v))
    grad_hidden = n * d * 2
    small = 4 << 20  # per-row fp32 coefficients and autograd's scalars
    print(f"backward extra {extra / 2**20:.1f} MiB: dlogits {dl_bytes / 2**20:.1f} + workspace "
          f"{ws_bytes / 2**20:.1f} + grad_hidden {grad_hidden / 2**20:.1f} MiB", flush=True)
    assert extra <= dl_bytes + ws_bytes + grad_hidden + small
    assert dl_bytes <= chunk * v * 4 + chunk * 32  # an fp32 [chunk, V] block


def test_repeated_runs_are_bit_identical(cuda):
    """No atomics: the per-tile partials, grad_hidden's vocabulary-range
    partial sums and the weight gradient's fp32 accumulation are all merged
    in a fixed order, so two runs give identical bits."""
    n, d, v = 2500, 512, 9000
    h, w, t, g_lp, g_ent = _inputs(n, d, v, seed=41)
    runs = []
    for _ in range(2):
        hc = h.to(cuda).requires_grad_()
        wc = w.to(cuda).requires_grad_()
        lp, ent = hip.fused_logprob_entropy(hc, wc, t.to(cuda), chunk=1024)
        (lp * g_lp.to(cuda) + ent * g_ent.to(cuda)).sum().backward()
        torch.cuda.synchronize()
        runs.append((lp.detach(), ent.detach(), hc.grad, wc.grad))
    for a, b, name in zip(runs[0], runs[1], ("lp", "ent", "grad hidden", "grad weight")):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("first_scored", [True, False])
def test_predictor_logprobs_match_the_streaming_gather(cuda, first_scored):
    """engine/streaming.py:4113-4130 / 5318-5349: predictors are
    cat([boundary, hidden[:-1]]) at the scored positions; the helper gathers
    only those rows.  Values and gradients (hidden, boundary) against the
    oracle applied to the reference's concatenation."""
    print(f"predictor_logprobs first_scored={first_scored}", flush=True)
    t, d, v = 300, 256, 4099
    g = torch.Generator().manual_seed(41 + first_scored)
    hidden = torch.randn(t, d, generator=g).to(torch.bfloat16)
    boundary = torch.randn(d, generator=g).to(torch.bfloat16)
    w = (torch.randn(v, d, generator=g) * 0.02).to(torch.bfloat16)
    tokens = torch.randint(0, v, (t,), generator=g).tolist()
    scored = (torch.rand(t, generator=g) < 0.6).tolist()
    scored[0] = first_scored
    pos = [j for j, s in enumerate(scored) if s]
    src = torch.cat([boundary.unsqueeze(0), hidden[:-1]])
    rows = src.index_select(0, torch.tensor(pos))
    tgt = torch.tensor([tokens[j] for j in pos])
    g_lp = torch.randn(len(pos), generator=g)
    want = ref.logprob_forward(rows, w, tgt, 1024)
    want_rows, _ = ref.logprob_backward(rows, w, tgt, g_lp, 1024)
    # scatter the per-row gradient back through the concatenation
    want_src = torch.zeros(t, d)
    want_src.index_add_(0, torch.tensor(pos), want_rows.float())
    hc = hidden.to(cuda).requires_grad_()
    bc = boundary.to(cuda).requires_grad_()
    lp = hip.predictor_logprobs(bc, hc, tokens, scored, w.to(cuda), chunk=64)
    (lp * g_lp.to(cuda)).sum().backward()
    torch.testing.assert_close(lp.cpu(), want, rtol=0, atol=1e-3)
    rel_close(hc.grad[:-1], want_src[1:], 1e-2, "grad hidden")
    assert torch.count_nonzero(hc.grad[-1]) == 0  # the last hidden predicts nothing here
    if first_scored:
        rel_close(bc.grad, want_src[0], 1e-2, "grad boundary")
    else:
        assert bc.grad is None or torch.count_nonzero(bc.grad) == 0
    # nothing scored: empty, on the weight's device
    empty = hip.predictor_logprobs(bc, hc, tokens, [False] * t, w.to(cuda))
    assert empty.shape == (0,) and empty.device == w.to(cuda).device
    with pytest.raises(ValueError, match="one entry per position"):
        hip.predictor_logprobs(bc, hc, tokens[:-1], scored, w.to(cuda))


def test_short_last_block_gets_a_large_enough_workspace(cuda):
    """A last dlogits block with fewer row tiles splits the vocabulary into
    more ranges than a full block and needs a larger grad-hidden workspace
    (3205 rows in blocks of 2048: 1157 rows, 4 ranges against 2); the
    backward sizes the workspace for both.  Rows are independent, so the
    oracle on sampled rows of both blocks is an exact check of them."""
    n, d, v, chunk = 3205, 4096, 16384, 1024
    assert hip.backward_block_rows(n, chunk) == 2048
    print(f"logprob short last block n={n} d={d} v={v}", flush=True)
    h, w, t, g_lp, g_ent = _inputs(n, d, v, seed=17)
    hc = h.to(cuda).requires_grad_()
    lp, ent = hip.fused_logprob_entropy(hc, w.to(cuda), t.to(cuda), chunk=chunk)
    (lp * g_lp.to(cuda) + ent * g_ent.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 2047, 2048, 2049, 2600, 3203, 3204])
    want_lp, want_ent = ref.logprob_entropy_forward(h[rows], w, t[rows], 1024)
    want_gh, _ = ref.logprob_entropy_backward(h[rows], w, t[rows], want_ent, g_lp[rows], g_ent[rows], 1024)
    torch.testing.assert_close(lp.cpu()[rows], want_lp, rtol=0, atol=1e-3)
    rel_close(hc.grad.cpu()[rows], want_gh, 1e-2, "grad hidden")
