"""Pin the attention and RMSNorm oracles (CPU)."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as ref
from oracle import forest as ofo
from oracle import rms_norm as rn


@pytest.mark.parametrize("t,s,hq,hkv", [(5, 5, 4, 4), (3, 11, 8, 2), (16, 40, 4, 1), (1, 9, 2, 2)])
def test_explicit_softmax_matches_torch_sdpa_lower_right(t, s, hq, hkv):
    g = torch.Generator().manual_seed(t * 100 + s)
    q = torch.randn(t, hq, 32, generator=g)
    k = torch.randn(s, hkv, 32, generator=g)
    v = torch.randn(s, hkv, 32, generator=g)
    out, lse = ref.bottom_right_attention(q, k, v, 0.2)
    want = ref.sdpa_lower_right(q, k, v, 0.2)
    torch.testing.assert_close(out, want, rtol=1e-5, atol=1e-5)
    # lse is the log-partition of the same masked scores
    kk = k.repeat_interleave(hq // hkv, 1)
    scores = torch.einsum("qhd,khd->hqk", q, kk) * 0.2
    mask = torch.arange(s)[None, :] <= (s - t) + torch.arange(t)[:, None]
    torch.testing.assert_close(lse, torch.logsumexp(scores.masked_fill(~mask, -math.inf), -1))


def test_gradcheck_fp64():
    g = torch.Generator().manual_seed(0)
    q = torch.randn(3, 2, 4, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(5, 1, 4, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(5, 1, 4, generator=g, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(
        lambda a, b, c: ref.bottom_right_attention(a, b, c, 0.5, dtype=torch.float64)[0], (q, k, v)
    )


def _group(n_traj, prompt_len, seed):
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, 900, (prompt_len,), generator=g).tolist()
    trajs = []
    for i in range(n_traj):
        segs = [ofo.Segment(tuple(prompt), "prompt", False)]
        for k in range(1 + i % 3):
            segs.append(ofo.Segment(tuple(torch.randint(0, 900, (4 + k + i,), generator=g).tolist()), "action", True))
            segs.append(ofo.Segment(tuple(torch.randint(0, 900, (7 + i,), generator=g).tolist()), "observation", False))
        trajs.append(ofo.Trajectory(segs, 0, i))
    return trajs


def test_forest_mask_equals_independent_per_trajectory_forward():
    """The reference's certification of sharing (tests/test_forest_attention.py:69-94)."""
    trajs = _group(5, 24, seed=3)
    forest = ofo.build_forest(trajs)
    plan = ofo.compile_plan(forest)
    p = len(plan["token_ids"])
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(p, h, 16, generator=g) for h in (4, 2, 2))
    mask = torch.tensor(ofo.visibility_mask(plan))
    shared = ref.masked_attention(q, k, v, mask)
    for t in trajs:
        path = []
        for n in forest.path_to_root(forest.leaf_of[t.traj_id]):
            path.extend(range(plan["node_start"][n], plan["node_end"][n]))
        idx = torch.tensor(path)
        alone, _ = ref.bottom_right_attention(q[idx], k[idx], v[idx])
        torch.testing.assert_close(shared[idx], alone, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_rms_norm_oracle_is_the_stock_module_bytes(dtype):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    torch.manual_seed(71)
    m = Qwen3RMSNorm(128, eps=1e-6).to(dtype)
    with torch.no_grad():
        m.weight.copy_(torch.linspace(0.4, 3.0, 128))
    x = torch.randn(64, 128).to(dtype)
    y, rstd = rn.rms_norm_forward(x, m.weight.detach(), 1e-6)
    assert torch.equal(y, m(x).detach())
    assert rstd.dtype == torch.float32 and rstd.shape == (64, 1)


def test_rms_norm_vjp_oracle_matches_closed_form():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(33, 96, generator=g)
    w = torch.linspace(0.4, 3.0, 96)
    dy = torch.randn(33, 96, generator=g)
    _, rstd = rn.rms_norm_forward(x, w, 1e-6)
    dx, dw = rn.rms_norm_backward(dy, x, w, 1e-6)
    cdx, cdw = rn.rms_norm_backward_closed_form(dy, x, w, rstd)
    torch.testing.assert_close(dx.double(), cdx, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(dw.double(), cdw, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("t,chunks,hq,hkv,n_keys,block", [(7, [9, 7], 8, 2, 9, 3), (40, [16, 40], 4, 1, 16, 512),
                                                          (5, [20], 2, 2, 11, 2)])
def test_prefix_key_grads_match_autograd(t, chunks, hq, hkv, n_keys, block):
    """The hand-written prefix-key VJP against autograd of chained_attention."""
    g = torch.Generator().manual_seed(t + hq)
    q = torch.randn(t, hq, 16, generator=g)
    ks = [torch.randn(n, hkv, 16, generator=g) for n in chunks]
    vs = [torch.randn(n, hkv, 16, generator=g) for n in chunks]
    dout = torch.randn(t, hq, 16, generator=g)
    _, _, gk, gv = ref.attention_with_grads(q, ks, vs, dout, 0.3, dtype=torch.float64)
    dk, dv = ref.prefix_key_grads(q, ks, vs, dout, 0.3, n_keys, rows_per_block=block, dtype=torch.float64)
    torch.testing.assert_close(dk, torch.cat(gk, 0)[:n_keys], rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dv, torch.cat(gv, 0)[:n_keys], rtol=1e-10, atol=1e-10)
