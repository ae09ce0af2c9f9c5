"""Fused-logprob oracle (CPU): the reference's chunk loop, restated.

Follows src/thundersync/accel/fused_logprob.py line for line in plain
PyTorch on the CPU: ``_matmul_accum`` (:44-58, the non-CUDA branch:
``.to(fp32)`` then mm), the forward chunk loop (:84-109 logprob, :255-263
with entropy) and the hand-written backward (:137-175, :279-297) including
the rounding of dlogits to the hidden dtype before the VJP GEMM, and the
fp32 weight-gradient accumulation cast once (:176-193, :298-307).
``gathered_logprobs`` / ``naive_logprobs`` restate :341-388.

Pinned by (tests/test_oracle_logprob.py): the dense closed form
``log_softmax(h W^T)[t]`` and ``H = -sum p log p`` (the reference's own
naive paths, tests/test_accel.py:33-65, tests/test_accel_entropy.py:170-177);
fp64 gradcheck of the hand-written backward; the reference's known-answer
precision cases (tests/test_accel_projection_precision.py:9-80); the
analytic entropy bounds 0 <= H <= log V.
"""

from __future__ import annotations

import torch

_ACCUM = {torch.bfloat16: torch.float32, torch.float16: torch.float32}


def _accum_dtype(dt):
    return _ACCUM.get(dt, dt)


def _matmul_accum(left, right):
    acc = _accum_dtype(left.dtype)
    return torch.mm(left.to(acc), right.to(acc))


def logprob_entropy_forward(hidden, weight, target, chunk=1024):
    """(logprob, entropy) per row, chunk by chunk (fused_logprob.py:250-263)."""
    n = hidden.shape[0]
    acc = _accum_dtype(hidden.dtype)
    out_lp = torch.empty(n, dtype=acc)
    out_ent = torch.empty(n, dtype=acc)
    for i in range(0, n, chunk):
        h = hidden[i : i + chunk]
        logits = _matmul_accum(h, weight.t())
        logits.sub_(logits.amax(dim=-1, keepdim=True))
        lse = torch.logsumexp(logits, dim=-1)
        picked = logits.gather(-1, target[i : i + chunk].unsqueeze(-1)).squeeze(-1)
        out_lp[i : i + chunk] = picked - lse
        probs = torch.softmax(logits, dim=-1)
        out_ent[i : i + chunk] = lse - (probs * logits).sum(-1)
    return out_lp, out_ent


def logprob_entropy_backward(hidden, weight, target, ent, grad_lp, grad_ent, chunk=1024,
                             needs_weight_grad=False):
    """(grad_hidden, grad_weight | None), fused_logprob.py:270-308."""
    n = hidden.shape[0]
    acc = _accum_dtype(hidden.dtype)
    grad_hidden = torch.zeros_like(hidden)
    grad_weight = torch.zeros_like(weight) if needs_weight_grad and n == 0 else None
    for i in range(0, n, chunk):
        h = hidden[i : i + chunk]
        t = target[i : i + chunk].unsqueeze(-1)
        g_lp = grad_lp[i : i + chunk].unsqueeze(-1)
        g_ent = grad_ent[i : i + chunk].unsqueeze(-1)
        logits = _matmul_accum(h, weight.t())
        logits.sub_(logits.amax(dim=-1, keepdim=True))
        logp = logits - torch.logsumexp(logits, dim=-1, keepdim=True)
        probs = logp.exp()
        hh = ent[i : i + chunk].unsqueeze(-1)
        dlogits = probs.mul_(-(g_lp + g_ent * (logp + hh)))
        dlogits.scatter_add_(-1, t, g_lp.to(acc))
        dlogits = dlogits.to(hidden.dtype)
        grad_hidden[i : i + chunk] = _matmul_accum(dlogits, weight).to(hidden.dtype)
        if needs_weight_grad:
            contribution = _matmul_accum(dlogits.t(), h)
            grad_weight = contribution if grad_weight is None else grad_weight.add_(contribution)
    if grad_weight is not None:
        grad_weight = grad_weight.to(weight.dtype)
    return grad_hidden, grad_weight


def logprob_forward(hidden, weight, target, chunk=1024):
    """Logprob only (fused_logprob.py:84-109)."""
    n = hidden.shape[0]
    out = torch.empty(n, dtype=_accum_dtype(hidden.dtype))
    for i in range(0, n, chunk):
        logits = _matmul_accum(hidden[i : i + chunk], weight.t())
        logits.sub_(logits.amax(dim=-1, keepdim=True))
        lse = torch.logsumexp(logits, dim=-1)
        picked = logits.gather(-1, target[i : i + chunk].unsqueeze(-1)).squeeze(-1)
        out[i : i + chunk] = picked - lse
    return out


def logprob_backward(hidden, weight, target, grad_out, chunk=1024, needs_weight_grad=False):
    """fused_logprob.py:116-194 (the logprob-only coefficient form)."""
    n = hidden.shape[0]
    grad_hidden = torch.zeros_like(hidden)
    grad_weight = torch.zeros_like(weight) if needs_weight_grad and n == 0 else None
    for i in range(0, n, chunk):
        h = hidden[i : i + chunk]
        t = target[i : i + chunk]
        g = grad_out[i : i + chunk].unsqueeze(-1)
        logits = _matmul_accum(h, weight.t())
        probs = torch.softmax(logits, dim=-1)
        probs.neg_()
        probs.scatter_add_(-1, t.unsqueeze(-1), torch.ones_like(g))
        dlogits = (probs * g).to(hidden.dtype)
        grad_hidden[i : i + chunk] = _matmul_accum(dlogits, weight).to(hidden.dtype)
        if needs_weight_grad:
            contribution = _matmul_accum(dlogits.t(), h)
            grad_weight = contribution if grad_weight is None else grad_weight.add_(contribution)
    if grad_weight is not None:
        grad_weight = grad_weight.to(weight.dtype)
    return grad_hidden, grad_weight


class FusedLogprobEntropy(torch.autograd.Function):
    """Autograd wrapper of the restated forward/backward (for gradcheck)."""

    @staticmethod
    def forward(ctx, hidden, weight, target, chunk):
        lp, ent = logprob_entropy_forward(hidden, weight, target, chunk)
        ctx.save_for_backward(hidden, weight, target, ent)
        ctx.chunk = chunk
        return lp, ent

    @staticmethod
    def backward(ctx, grad_lp, grad_ent):
        hidden, weight, target, ent = ctx.saved_tensors
        gh, gw = logprob_entropy_backward(hidden, weight, target, ent, grad_lp, grad_ent, ctx.chunk,
                                          needs_weight_grad=ctx.needs_input_grad[1])
        return gh, gw, None, None


def naive_logprob_entropy(hidden, weight, target):
    """Dense closed form: the whole [N, V] block, autograd for the backward."""
    acc = _accum_dtype(hidden.dtype)
    logits = torch.nn.functional.linear(hidden.to(acc), weight.to(acc))
    logp = torch.log_softmax(logits, dim=-1)
    lp = logp.gather(-1, target.unsqueeze(-1)).squeeze(-1)
    ent = -(logp.exp() * logp).sum(-1)
    return lp, ent


def gathered_logprobs(hidden, weight, token_ids, loss_mask, chunk=1024):
    """fused_logprob.py:341-367 over the restated forward."""
    n = token_ids.shape[0]
    idx = loss_mask.nonzero(as_tuple=True)[0]
    idx = idx[idx > 0]
    if idx.numel() == 0:
        return torch.zeros(n, dtype=_accum_dtype(hidden.dtype))
    lp = logprob_forward(hidden[idx - 1], weight, token_ids[idx], chunk)
    return torch.zeros(n, dtype=lp.dtype).index_put((idx,), lp)
