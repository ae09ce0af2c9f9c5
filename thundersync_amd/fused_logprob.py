"""Fused chunked-vocab logprob / entropy on the gfx950 kernels.

Drop-in for the reference's ``accel/fused_logprob.py:197-367``: same
signatures, same validation errors, same outputs (fp32 ``[N]``), same
gradient semantics -- gradient with respect to ``hidden`` always, with
respect to ``weight`` only when ``weight.requires_grad``.

Forward: ``ts_logprob_fwd`` computes logits tile by tile on MFMA and reduces
them in the GEMM epilogue; no ``[N, V]`` or ``[chunk, V]`` logit block is
ever stored.  It returns logprob, entropy and the per-row log-sum-exp, which
the backward reuses instead of recomputing the row statistics.

Backward, per block of two chunks of rows (the reference's chunk loop,
FL:143-193, with its O(chunk * V) memory: a bf16 block of two chunks is the
size of the reference's fp32 logit block of one): ``ts_logprob_dlogits`` recomputes
the logits and writes the block's bf16 dlogits (rounded to bf16 as the
reference rounds its dlogits to the hidden dtype, FL:165 and :295);
``ts_logprob_grad_hidden`` multiplies them by the weight, read in place;
when the head is trainable ``ts_logprob_grad_weight`` adds ``dl^T h`` into
an fp32 accumulator, cast once at the end (FL:176-193).  Extra device memory
is the ``[chunk, V]`` bf16 dlogits block plus a workspace of vocabulary-range
partial sums for grad_hidden when one block's row tiles do not fill the GPU,
and the fp32 ``[V, D]`` accumulator when the weight gradient is needed.

bf16 or fp16 (one element type per call) on the MFMA kernels above; fp32
and fp64 at their own precision, as the reference keeps them (FL:27-58):
logits, statistics, dlogits and both VJP products in the input type on the
vector-ALU kernels (``ts_logprob_fwd_exact``, ``ts_logprob_dlogits_exact``,
``ts_matmul_exact``), with the same O(chunk * V) dlogits block and outputs
in the input type.  GPU only: other dtypes and CPU tensors raise.
"""

from __future__ import annotations

import torch

from . import _lib
from .operator_profiling import device_role, operator_range


ELEMENT_DTYPES = (torch.bfloat16, torch.float16)  # the MFMA kernels
EXACT_DTYPES = (torch.float32, torch.float64)     # the input-precision kernels
CHECK_TARGETS_ENV = "THUNDERSYNC_CHECK_TARGETS"


def _check_targets(target: torch.Tensor, vocab: int) -> None:
    """With THUNDERSYNC_CHECK_TARGETS=1, refuse targets outside [0, vocab),
    naming the first offending row (costs one device synchronisation).

    Without it an out-of-range target is not an error, as it is in the
    reference's gather: its logprob comes back NaN and its dlogits row gets
    no one-hot term (every vocabulary entry takes its -p g part), so a bad
    token id surfaces as a NaN loss."""
    import os

    if os.environ.get(CHECK_TARGETS_ENV, "0") in ("", "0") or target.numel() == 0:
        return
    bad = ((target < 0) | (target >= vocab)).nonzero()
    if bad.numel():
        row = int(bad[0, 0])
        raise ValueError(f"target[{row}] = {int(target[row])} is outside the vocabulary [0, {vocab})")


def _validate(hidden: torch.Tensor, weight: torch.Tensor, target: torch.Tensor) -> None:
    # the reference's contract, accel/fused_logprob.py:209-216
    if hidden.dim() != 2:
        raise ValueError(f"hidden must be [N, D], got {tuple(hidden.shape)}")
    if target.shape[0] != hidden.shape[0]:
        raise ValueError("target must have one entry per hidden row")
    if weight.shape[1] != hidden.shape[1]:
        raise ValueError(f"weight {tuple(weight.shape)} does not match hidden dim {hidden.shape[1]}")
    if not hidden.is_cuda or not weight.is_cuda or not target.is_cuda:
        raise RuntimeError("thundersync_amd fused logprob runs on the GPU only; got a CPU tensor")
    if hidden.dtype not in ELEMENT_DTYPES + EXACT_DTYPES or weight.dtype != hidden.dtype:
        raise TypeError(
            "thundersync_amd fused logprob takes bf16, fp16, fp32 or fp64 hidden and weight of one dtype, got "
            f"{hidden.dtype}/{weight.dtype}"
        )
    _check_targets(target, weight.shape[0])


def _pad_dim(t: torch.Tensor) -> torch.Tensor:
    """Zero-pad the hidden dim to a multiple of 8 (the logits are unchanged)."""
    pad = (-t.shape[1]) % 8
    return torch.nn.functional.pad(t, (0, pad)) if pad else t


def _rows_ok(t: torch.Tensor) -> torch.Tensor:
    if t.stride(1) == 1 and t.stride(0) % 8 == 0 and t.data_ptr() % 16 == 0:
        return t
    return t.contiguous()


def _unit_stride(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(1) == 1 or t.shape[1] <= 1 else t.contiguous()


def _forward_exact(hidden, weight, target, with_entropy):
    """fp32 / fp64: logprob, entropy and lse in the input type."""
    lib = _lib.require_library()
    h, w = _unit_stride(hidden), _unit_stride(weight)
    t = target.to(torch.int64).contiguous()
    n, d = h.shape
    v = w.shape[0]
    code = _lib.dtype_code(h.dtype)
    lp = torch.empty(n, dtype=h.dtype, device=h.device)
    lse = torch.empty(n, dtype=h.dtype, device=h.device)
    ent = torch.empty(n, dtype=h.dtype, device=h.device) if with_entropy else None
    ws_bytes = int(lib.ts_logprob_fwd_exact_workspace(n, v, code))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=h.device)
    _lib.check(
        lib.ts_logprob_fwd_exact(
            h.data_ptr(), max(h.stride(0), d), w.data_ptr(), max(w.stride(0), d), t.data_ptr(), n, d, v,
            lp.data_ptr(), _lib.ptr(ent), lse.data_ptr(), ws.data_ptr(), ws_bytes, code, _lib.stream_of(h),
        ),
        f"ts_logprob_fwd_exact(rows={n}, dim={d}, vocab={v}, {h.dtype})",
    )
    return lp, ent, lse


def _backward_exact(hidden, weight, target, lse, ent, grad_lp, grad_ent, chunk, needs_weight_grad):
    """fp32 / fp64: the reference's chunk loop (FL:137-193) with a [chunk, V]
    dlogits block in the input type; grad_weight accumulated in it."""
    lib = _lib.require_library()
    h, w = _unit_stride(hidden), _unit_stride(weight)
    t = target.to(torch.int64).contiguous()
    n, d = h.shape
    v = w.shape[0]
    dt, dev = h.dtype, h.device
    grad_hidden = torch.empty(n, d, dtype=dt, device=dev)
    grad_weight = torch.zeros(v, d, dtype=dt, device=dev) if needs_weight_grad else None
    if n == 0:
        return grad_hidden, grad_weight
    code, stream = _lib.dtype_code(dt), _lib.stream_of(h)
    ldh, ldw = max(h.stride(0), d), max(w.stride(0), d)
    block = min(max(1, int(chunk)), n)
    dl = torch.empty(block, v, dtype=dt, device=dev)
    g_lp = grad_lp.to(dt).contiguous()
    g_ent = grad_ent.to(dt).contiguous() if grad_ent is not None else None
    esize = h.element_size()
    for i in range(0, n, block):
        rows = min(block, n - i)
        h_i = h.data_ptr() + i * ldh * esize
        with operator_range("logprob_head_coefficient_backward", role=device_role(dev), rows=rows, vocab=v):
            _lib.check(
                lib.ts_logprob_dlogits_exact(
                    h_i, ldh, w.data_ptr(), ldw, t[i:].data_ptr(), lse[i:].data_ptr(),
                    ent[i:].data_ptr() if g_ent is not None else None, g_lp[i:].data_ptr(),
                    g_ent[i:].data_ptr() if g_ent is not None else None, rows, d, v, dl.data_ptr(), v, code, stream,
                ),
                f"ts_logprob_dlogits_exact(rows={rows}, dim={d}, vocab={v})",
            )
        with operator_range("logprob_head_hidden_vjp", role=device_role(dev), rows=rows, hidden=d, vocab=v):
            # grad_hidden[i:i+rows] = dl . W
            _lib.check(
                lib.ts_matmul_exact(dl.data_ptr(), v, 1, w.data_ptr(), ldw, 1, rows, d, v,
                                    grad_hidden[i:].data_ptr(), d, 0, code, stream),
                f"ts_matmul_exact(dlogits . weight, rows={rows}, dim={d}, vocab={v})",
            )
        if grad_weight is not None:
            with operator_range("logprob_head_weight_vjp", role=device_role(dev), rows=rows, hidden=d, vocab=v):
                # grad_weight += dl^T . h[i:i+rows]
                _lib.check(
                    lib.ts_matmul_exact(dl.data_ptr(), 1, v, h_i, ldh, 1, v, d, rows,
                                        grad_weight.data_ptr(), d, 1, code, stream),
                    f"ts_matmul_exact(dlogits^T . hidden, rows={rows}, dim={d}, vocab={v})",
                )
    return grad_hidden, grad_weight


def _forward(hidden, weight, target, with_entropy):
    if hidden.dtype in EXACT_DTYPES:
        return _forward_exact(hidden, weight, target, with_entropy)
    lib = _lib.require_library()
    h, w = _rows_ok(_pad_dim(hidden)), _rows_ok(_pad_dim(weight))
    t = target.to(torch.int64).contiguous()
    n, d = h.shape
    v = w.shape[0]
    lp = torch.empty(n, dtype=torch.float32, device=h.device)
    lse = torch.empty(n, dtype=torch.float32, device=h.device)
    ent = torch.empty(n, dtype=torch.float32, device=h.device) if with_entropy else None
    ws_bytes = int(lib.ts_logprob_fwd_workspace(n, v))
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=h.device)
    _lib.check(
        lib.ts_logprob_fwd(
            h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0), t.data_ptr(), n, d, v,
            lp.data_ptr(), _lib.ptr(ent), lse.data_ptr(), ws.data_ptr(), ws_bytes,
            _lib.dtype_code(h.dtype), _lib.stream_of(h),
        ),
        f"ts_logprob_fwd(rows={n}, dim={d}, vocab={v})",
    )
    return lp, ent, lse


# Rows of a dlogits block, in chunks: the reference's chunk loop holds an fp32
# [chunk, V] logit block at a time (FL:137-175); a bf16 dlogits block of
# BLOCK_CHUNKS = 2 chunks takes the same bytes, and its launches end in a
# partial round of work-groups half as often as one-chunk blocks would.
BLOCK_CHUNKS = 2


def backward_block_rows(n: int, chunk: int) -> int:
    """Rows per dlogits block: ``BLOCK_CHUNKS * chunk`` (at least one row),
    rounded down to a multiple of 256 (whole GEMM tiles) when that stays
    positive, and never more than the rows there are."""
    block = max(1, BLOCK_CHUNKS * int(chunk))
    if block >= 256:
        block -= block % 256
    return min(block, max(n, 1))


def _backward(hidden, weight, target, lse, ent, grad_lp, grad_ent, chunk, needs_weight_grad):
    if hidden.dtype in EXACT_DTYPES:
        return _backward_exact(hidden, weight, target, lse, ent, grad_lp, grad_ent, chunk, needs_weight_grad)
    lib = _lib.require_library()
    d_in = hidden.shape[1]
    h, w = _rows_ok(_pad_dim(hidden)), _rows_ok(_pad_dim(weight))
    t = target.to(torch.int64).contiguous()
    n, d = h.shape
    v = w.shape[0]
    vp = (v + 7) // 8 * 8
    grad_hidden = torch.empty_like(h)
    grad_weight = torch.zeros(v, d, dtype=torch.float32, device=h.device) if needs_weight_grad else None
    if n == 0:
        return grad_hidden[:, :d_in], (grad_weight[:, :d_in].to(weight.dtype) if grad_weight is not None else None)
    stream = _lib.stream_of(h)
    code = _lib.dtype_code(h.dtype)
    block = backward_block_rows(n, chunk)
    dl = torch.empty(block, vp, dtype=w.dtype, device=w.device)
    # the last block may be shorter, and fewer row tiles take more vocabulary
    # ranges: size the workspace for whichever of the two block sizes needs more
    tail = n % block
    ws_bytes = max(int(lib.ts_logprob_grad_hidden_workspace(rows, d, v)) for rows in {block, tail or block})
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=h.device)
    g_lp = grad_lp.to(torch.float32).contiguous()
    g_ent = grad_ent.to(torch.float32).contiguous() if grad_ent is not None else None
    for i in range(0, n, block):
        rows = min(block, n - i)
        hi = h[i : i + rows]
        with operator_range("logprob_head_coefficient_backward", role=device_role(h.device), rows=rows, vocab=v):
            _lib.check(
                lib.ts_logprob_dlogits(
                    hi.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0), t[i:].data_ptr(),
                    lse[i:].data_ptr(), ent[i:].data_ptr() if ent is not None else None,
                    g_lp[i:].data_ptr(), g_ent[i:].data_ptr() if g_ent is not None else None,
                    rows, d, v, dl.data_ptr(), vp, code, stream,
                ),
                f"ts_logprob_dlogits(rows={rows}, dim={d}, vocab={v})",
            )
        with operator_range("logprob_head_hidden_vjp", role=device_role(h.device), rows=rows, hidden=d, vocab=v):
            _lib.check(
                lib.ts_logprob_grad_hidden(
                    dl.data_ptr(), vp, w.data_ptr(), w.stride(0), rows, d, v,
                    grad_hidden[i:].data_ptr(), grad_hidden.stride(0), ws.data_ptr(), ws_bytes, code, stream,
                ),
                f"ts_logprob_grad_hidden(rows={rows}, dim={d}, vocab={v})",
            )
        if grad_weight is not None:
            # fp32 accumulation across blocks, cast once (FL:176-193)
            with operator_range("logprob_head_weight_vjp", role=device_role(h.device), rows=rows, hidden=d, vocab=v):
                _lib.check(
                    lib.ts_logprob_grad_weight(
                        dl.data_ptr(), vp, hi.data_ptr(), h.stride(0), rows, d, v,
                        grad_weight.data_ptr(), grad_weight.stride(0), code, stream,
                    ),
                    f"ts_logprob_grad_weight(rows={rows}, dim={d}, vocab={v})",
                )
    if d != d_in:
        grad_hidden = grad_hidden[:, :d_in].contiguous()
        grad_weight = grad_weight[:, :d_in] if grad_weight is not None else None
    return grad_hidden, (grad_weight.to(weight.dtype) if grad_weight is not None else None)


class _FusedLinearLogprob(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, target, chunk, needs_weight_grad):
        with operator_range("fused_logprob_forward", role=device_role(hidden.device), tokens=hidden.shape[0],
                            hidden=hidden.shape[1], vocab=weight.shape[0], dtype=hidden.dtype):
            lp, _ent, lse = _forward(hidden, weight, target, False)
        ctx.save_for_backward(hidden, weight, target, lse)
        ctx.chunk, ctx.needs_weight_grad = chunk, needs_weight_grad
        return lp

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        hidden, weight, target, lse = ctx.saved_tensors
        with operator_range("fused_logprob_backward", role=device_role(hidden.device), tokens=hidden.shape[0],
                            hidden=hidden.shape[1], vocab=weight.shape[0], weight_grad=ctx.needs_weight_grad):
            gh, gw = _backward(hidden, weight, target, lse, None, grad_out, None, ctx.chunk, ctx.needs_weight_grad)
        return gh, gw, None, None, None


class _FusedLinearLogprobEntropy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, target, chunk, needs_weight_grad):
        with operator_range("fused_logprob_entropy_forward", role=device_role(hidden.device),
                            tokens=hidden.shape[0], hidden=hidden.shape[1], vocab=weight.shape[0]):
            lp, ent, lse = _forward(hidden, weight, target, True)
        ctx.save_for_backward(hidden, weight, target, lse, ent)
        ctx.chunk, ctx.needs_weight_grad = chunk, needs_weight_grad
        return lp, ent

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_lp, grad_ent):
        hidden, weight, target, lse, ent = ctx.saved_tensors
        with operator_range("fused_logprob_entropy_backward", role=device_role(hidden.device),
                            tokens=hidden.shape[0], hidden=hidden.shape[1], vocab=weight.shape[0]):
            gh, gw = _backward(hidden, weight, target, lse, ent, grad_lp, grad_ent, ctx.chunk,
                               ctx.needs_weight_grad)
        return gh, gw, None, None, None


def fused_logprob(hidden: torch.Tensor, weight: torch.Tensor, target: torch.Tensor, *, chunk: int = 1024):
    """Per-position log pi(target | context) without materialising ``[N, V]``."""
    _validate(hidden, weight, target)
    return _FusedLinearLogprob.apply(hidden, weight, target, chunk, weight.requires_grad)


def fused_logprob_entropy(hidden: torch.Tensor, weight: torch.Tensor, target: torch.Tensor, *,
                          chunk: int = 1024):
    """Per-position (logprob, entropy of the full-vocabulary distribution)."""
    _validate(hidden, weight, target)
    return _FusedLinearLogprobEntropy.apply(hidden, weight, target, chunk, weight.requires_grad)


def gathered_logprobs(hidden: torch.Tensor, weight: torch.Tensor, token_ids: torch.Tensor,
                      loss_mask: torch.Tensor, *, chunk: int = 1024) -> torch.Tensor:
    """Logprobs laid back out over the sequence, zero where not needed (FL:341-367).

    Position k is predicted from position k-1's hidden state; position 0 is
    never scored.  Projection happens only for masked positions.
    """
    n = token_ids.shape[0]
    idx = loss_mask.nonzero(as_tuple=True)[0]
    idx = idx[idx > 0]
    if idx.numel() == 0:
        return torch.zeros(n, dtype=torch.float32, device=hidden.device)
    lp = fused_logprob(hidden[idx - 1], weight, token_ids[idx], chunk=chunk)
    out = torch.zeros(n, dtype=lp.dtype, device=lp.device)
    return out.index_put((idx,), lp)


def predictor_logprobs(boundary_hidden: torch.Tensor, hidden: torch.Tensor, tokens, scored, weight: torch.Tensor,
                       *, chunk: int = 1024) -> torch.Tensor:
    """Logprobs of a chunk's scored tokens, each predicted by the hidden state
    one position earlier; the chunk's first position by ``boundary_hidden``,
    the last hidden state of what precedes the chunk.

    The logprob gathers of the reference's streaming engine: appended turns
    (engine/streaming.py:4113-4130, the previous chunk's last hidden) and
    suffix rebuilds (:5318-5349, the prompt's last hidden).  There the
    predictors are ``cat([boundary, hidden[:-1]])`` indexed at the scored
    positions; here only the scored predictor rows are gathered (no ``[T, D]``
    copy), and gradients reach ``hidden``, ``boundary_hidden`` and, when it
    requires them, ``weight``.  ``tokens`` and ``scored`` are per-position
    sequences (Python or 1-D tensors); the result is fp32 ``[n_scored]`` in
    position order, empty when nothing is scored.
    """
    t = hidden.shape[0]
    if boundary_hidden.shape != hidden.shape[1:]:
        raise ValueError(f"boundary_hidden {tuple(boundary_hidden.shape)} must be one row of {tuple(hidden.shape)}")
    scored_t = torch.as_tensor(scored, dtype=torch.bool).cpu()
    tokens_t = torch.as_tensor(tokens, dtype=torch.long).cpu()
    if scored_t.shape != (t,) or tokens_t.shape != (t,):
        raise ValueError(f"tokens and scored need one entry per position ({t})")
    positions = scored_t.nonzero(as_tuple=True)[0]
    if positions.numel() == 0:
        return torch.zeros(0, dtype=torch.float32, device=weight.device)
    dev = hidden.device
    first = bool(positions[0] == 0)
    rest = positions[1:] if first else positions
    rows = hidden.index_select(0, (rest - 1).to(dev, non_blocking=True))
    if first:
        rows = torch.cat([boundary_hidden.unsqueeze(0), rows], dim=0)
    target = tokens_t.index_select(0, positions).to(dev, non_blocking=True)
    return fused_logprob(rows, weight, target, chunk=chunk)
