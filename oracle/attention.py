"""Attention oracle (CPU, fp32 or fp64).

Restates the reference's masked path: ``F.scaled_dot_product_attention`` with
``attn_mask=causal_lower_right(T, S)`` and GQA by ``repeat_interleave``
(src/thundersync/engine/streaming.py:1146-1162), written out as an explicit
softmax, and the dense forest reference (engine/attention.py:234-257 with
engine/plan.py:343-362).  Gradients come from autograd of these formulas.

Pinned by (tests/test_oracle_attention.py): torch's own SDPA with
``causal_lower_right`` on the CPU (an independent implementation of the same
mask); the forest mask against an independent per-trajectory causal forward
(tests/test_forest_attention.py:69-94 of the reference); fp64 gradcheck of the
explicit softmax.
"""

from __future__ import annotations

import math

import torch


def bottom_right_attention(q, k, v, scale=None, *, dtype=torch.float32):
    """q ``[T, Hq, D]``, k/v ``[S, Hkv, D]`` -> (out ``[T, Hq, D]``, lse ``[Hq, T]``).

    Query i sees keys ``0 .. S - T + i`` (bottom-right-aligned causal).
    Computed in ``dtype``; differentiable.
    """
    t, hq, d = q.shape
    s, hkv = k.shape[0], k.shape[1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    if hq != hkv:
        k = k.repeat_interleave(hq // hkv, dim=1)
        v = v.repeat_interleave(hq // hkv, dim=1)
    scores = torch.einsum("qhd,khd->hqk", q.to(dtype), k.to(dtype)) * scale
    qi = torch.arange(t).unsqueeze(1)
    kj = torch.arange(s).unsqueeze(0)
    visible = kj <= (s - t) + qi
    scores = scores.masked_fill(~visible.unsqueeze(0), float("-inf"))
    lse = torch.logsumexp(scores, dim=-1)
    probs = torch.softmax(scores, dim=-1)
    out = torch.einsum("hqk,khd->qhd", probs, v.to(dtype))
    return out, lse


def chained_attention(q, ks, vs, scale=None, *, dtype=torch.float32):
    """``_causal_sdpa`` over chunk lists: cat(ks), cat(vs), bottom-right causal."""
    return bottom_right_attention(q, torch.cat(list(ks), 0), torch.cat(list(vs), 0), scale, dtype=dtype)


def sdpa_lower_right(q, k, v, scale):
    """The reference's own masked call on the CPU (streaming.py:1146-1162)."""
    from torch.nn.attention.bias import causal_lower_right
    import torch.nn.functional as F

    qt = q.transpose(0, 1).unsqueeze(0)
    kt = k.transpose(0, 1).unsqueeze(0)
    vt = v.transpose(0, 1).unsqueeze(0)
    n_rep = qt.shape[1] // kt.shape[1]
    if n_rep > 1:
        kt = kt.repeat_interleave(n_rep, dim=1)
        vt = vt.repeat_interleave(n_rep, dim=1)
    out = F.scaled_dot_product_attention(
        qt, kt, vt, attn_mask=causal_lower_right(qt.shape[2], kt.shape[2]), scale=scale
    )
    return out[0].transpose(0, 1)


def masked_attention(q, k, v, mask, scale=None, *, dtype=torch.float32):
    """Dense attention over a ``[P, P]`` bool visibility mask (engine/attention.py:234-257)."""
    hq, hkv = q.shape[1], k.shape[1]
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    if hq != hkv:
        k = k.repeat_interleave(hq // hkv, dim=1)
        v = v.repeat_interleave(hq // hkv, dim=1)
    scores = torch.einsum("qhd,khd->hqk", q.to(dtype), k.to(dtype)) * scale
    scores = scores.masked_fill(~mask.unsqueeze(0), float("-inf"))
    return torch.einsum("hqk,khd->qhd", scores.softmax(dim=-1), v.to(dtype))


def attention_with_grads(q, ks, vs, dout, scale, *, dtype=torch.float32):
    """(out, dq, [dk...], [dv...]) of chained_attention in ``dtype``."""
    qq = q.detach().to(dtype).requires_grad_()
    kk = [k.detach().to(dtype).requires_grad_() for k in ks]
    vv = [v.detach().to(dtype).requires_grad_() for v in vs]
    out, _ = chained_attention(qq, kk, vv, scale, dtype=dtype)
    grads = torch.autograd.grad(out, [qq, *kk, *vv], dout.to(dtype))
    n = len(ks)
    return out.detach(), grads[0], list(grads[1 : 1 + n]), list(grads[1 + n :])


def prefix_key_grads(q, ks, vs, dout, scale, n_keys, *, rows_per_block=512, dtype=torch.float32):
    """(dk, dv) of the first ``n_keys`` keys of ``chained_attention(q, ks, vs)``.

    The same bottom-right-causal softmax attention as :func:`chained_attention`,
    differentiated by hand for the keys of a shared prefix only (the keys a
    prompt run contributes to every segment that reads it), query rows a block
    at a time so that long segments fit in memory:
    ``P = softmax(scale Q K^T)``, ``O = P V``, ``delta = rowsum(dO * O)``,
    ``dV[:n] = P[:, :n]^T dO``, ``dK[:n] = scale (P[:, :n] * (dO V[:n]^T - delta))^T Q``.
    Returns fp32/``dtype`` tensors ``[n_keys, Hkv, D]``.
    """
    k = torch.cat(list(ks), 0).to(dtype)
    v = torch.cat(list(vs), 0).to(dtype)
    t, hq, d = q.shape
    s, hkv = k.shape[0], k.shape[1]
    group = hq // hkv
    # [Hkv, group, rows, D] views of the queries; keys [Hkv, S, D]
    kh = k.permute(1, 0, 2).contiguous()
    vh = v.permute(1, 0, 2).contiguous()
    dk = torch.zeros(hkv, n_keys, d, dtype=dtype)
    dv = torch.zeros(hkv, n_keys, d, dtype=dtype)
    for r0 in range(0, t, rows_per_block):
        r1 = min(t, r0 + rows_per_block)
        qb = q[r0:r1].to(dtype).reshape(r1 - r0, hkv, group, d).permute(1, 2, 0, 3).contiguous()
        gb = dout[r0:r1].to(dtype).reshape(r1 - r0, hkv, group, d).permute(1, 2, 0, 3).contiguous()
        scores = torch.matmul(qb, kh.unsqueeze(1).transpose(-1, -2).contiguous()) * scale
        rows = torch.arange(r0, r1)[:, None]
        visible = torch.arange(s)[None, :] <= (s - t) + rows
        scores = scores.masked_fill(~visible, float("-inf"))
        p = torch.softmax(scores, dim=-1)
        out = torch.matmul(p, vh.unsqueeze(1))
        delta = (gb * out).sum(-1, keepdim=True)
        pp = p[..., :n_keys]
        dpp = torch.matmul(gb, vh[:, :n_keys].unsqueeze(1).transpose(-1, -2).contiguous())
        ds = pp * (dpp - delta)
        dv += torch.matmul(pp.transpose(-1, -2), gb).sum(1)
        dk += torch.matmul(ds.transpose(-1, -2), qb).sum(1) * scale
    return dk.permute(1, 0, 2).contiguous(), dv.permute(1, 0, 2).contiguous()
