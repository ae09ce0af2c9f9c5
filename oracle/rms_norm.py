"""RMSNorm oracle (CPU).

Restates accel/rms_norm.py:9-17 (forward: ``x = h.float(); rstd =
rsqrt(mean(x^2) + eps); y = w * (x * rstd).to(dtype)``) and the FP32 VJP of
accel/rms_norm.py:33-38 (autograd of ``F.rms_norm`` in fp32 on the CPU).

``device_forward`` restates the same forward as the GPU computes it: the
reference's primal is "the original primal bytes" of the stock module
(accel/rms_norm.py:46-52, tests/test_rms_norm_precision.py:27-39), and on the
GPU those bytes come from torch's reduction kernel (third-party: torch
2.10.0+rocm7.0, ATen/native/hip/Reduce.cuh -- setReduceConfig,
input_vectorized_thread_reduce_impl, thread_reduce_impl, block_x_reduce,
block_y_reduce, MeanOps) summing ``x.pow(2)`` in a fixed, shape-dependent
order, and from ``torch.rsqrt``, which is correctly rounded in fp32.

Pinned by: the forward against transformers' stock ``Qwen3RMSNorm`` (bytes
equal, the reference's own claim, tests/test_rms_norm_precision.py:27-39);
``device_forward`` bit for bit against stock-module outputs recorded on an
MI355X (tests/golden/rmsnorm_device.npz, written by
tests/golden/make_rmsnorm_golden.py) and within fp32 rounding of an fp64
sum; the VJP against an fp64 autograd of the unrounded formula and against
the closed form ``dx = rstd*(g - xhat*mean(g*xhat))``, ``dw = sum(dy*xhat)``.
"""

from __future__ import annotations

import numpy as np
import torch


def rms_norm_forward(hidden: torch.Tensor, weight: torch.Tensor, eps: float):
    """accel/rms_norm.py:11-14. Returns (primal, rstd[..., 1] fp32)."""
    x = hidden.to(torch.float32)
    variance = x.pow(2).mean(-1, keepdim=True)
    rstd = torch.rsqrt(variance + eps)
    primal = weight * (x * rstd).to(hidden.dtype)
    return primal, rstd


def rms_norm_backward(gradient, hidden, weight, eps: float):
    """accel/rms_norm.py:33-38: autograd of F.rms_norm in fp32.

    Returns (dx in hidden.dtype, dw in weight.dtype).
    """
    with torch.enable_grad():
        x = hidden.detach().float().requires_grad_()
        w = weight.detach().float().requires_grad_()
        out = torch.nn.functional.rms_norm(x, tuple(weight.shape), w, eps)
        dx, dw = torch.autograd.grad(out, (x, w), gradient.float())
    return dx.to(hidden.dtype), dw.to(weight.dtype)


def rms_norm_backward_closed_form(gradient, hidden, weight, rstd):
    """The VJP written out, in fp64, from the saved statistic (for pinning)."""
    x = hidden.double()
    r = rstd.double()
    g = gradient.double() * weight.double()
    xhat = x * r
    dot = (g * xhat).mean(-1, keepdim=True)
    dx = r * (g - xhat * dot)
    dw = (gradient.double() * xhat).reshape(-1, hidden.shape[-1]).sum(0)
    return dx, dw


# ---------------------------------------------------------------------------
# the forward as the GPU computes it
# ---------------------------------------------------------------------------
_F32 = np.float32


def _last_pow2(n: int) -> int:
    return 1 << (int(n).bit_length() - 1)


def device_reduce_schedule(rows: int, width: int, num_cu: int = 256):
    """setReduceConfig (Reduce.cuh) for summing the contiguous last dim of a
    [rows, width] fp32 tensor: (vec, bw, bh, ym, step).

    Thread (x, y) of bw x bh sums loads x + y*ym, + step, ...; vec means
    4-element vector loads (width >= 128).  Returns None where torch would
    split one row over several work-groups (not restated).
    """
    max_threads, warp = 512, 64
    vec = width >= 128
    dim0 = width // 4 if vec else width
    d0 = _last_pow2(dim0) if dim0 < max_threads else max_threads
    d1 = _last_pow2(rows) if rows < max_threads else max_threads
    bw = min(d0, warp)
    block_h = min(d1, max_threads // bw)
    bw = min(d0, max_threads // block_h)
    step = bw
    per_thread = -(-width // step)
    split = per_thread >= min(block_h * 16, 256)
    if rows > 1 and per_thread < 1024 and num_cu < 100:
        split = False
    bh, ym = 1, 0
    if split:
        ym, step, bh = step, step * block_h, block_h
        if rows == 1 and -(-width // step) >= 256:
            return None
    return vec, bw, bh, ym, step


def _thread_sum(sq, width, x, y, sched, shift):
    """One reduction thread's sum over rows `sq` [n, width] (float32)."""
    vec, bw, bh, ym, step = sched
    n = sq.shape[0]
    acc = [np.zeros(n, _F32) for _ in range(4)]
    tail_ok = bh == 1 or y == 0
    if vec:
        end, d0 = width, 0
        if shift > 0:
            d0, end = -shift, width + shift
            if shift <= x < 4 and tail_ok:
                acc[0] = (acc[0] + sq[:, d0 + x]).astype(_F32)
            end, d0 = end - 4, d0 + 4
        idx = x + y * ym
        while idx * 4 + 3 < end:
            for i in range(4):
                acc[i] = (acc[i] + sq[:, d0 + idx * 4 + i]).astype(_F32)
            idx += step
        tail = end - end % 4 + x
        if tail_ok and tail < end:
            acc[0] = (acc[0] + sq[:, d0 + tail]).astype(_F32)
    else:
        idx = x + y * ym
        while idx + 3 * step < width:
            for i in range(4):
                acc[i] = (acc[i] + sq[:, idx + i * step]).astype(_F32)
            idx += 4 * step
        for i in range(4):
            if idx >= width:
                break
            acc[i] = (acc[i] + sq[:, idx]).astype(_F32)
            idx += step
    s = acc[0]
    for i in range(1, 4):
        s = (s + acc[i]).astype(_F32)
    return s


def device_row_sums(x: np.ndarray, rows: int | None = None, row_index=None, num_cu: int = 256):
    """sum(x**2, -1) of fp32 rows in the order torch's GPU reduction uses.

    ``x`` is [n, width]; ``rows`` is the row count of the whole tensor the
    rows came from (it sets the schedule) and ``row_index`` their indices in
    it (they set each row's offset from a 16-byte boundary); by default the
    rows are the whole tensor.
    """
    x = np.ascontiguousarray(x, dtype=_F32)
    n, width = x.shape
    rows = n if rows is None else rows
    row_index = np.arange(n) if row_index is None else np.asarray(row_index)
    sched = device_reduce_schedule(rows, width, num_cu)
    if sched is None:
        raise ValueError(f"width {width}: one row summed across work-groups; not restated")
    vec, bw, bh, _, _ = sched
    sq = (x * x).astype(_F32)
    out = np.zeros(n, _F32)
    shifts = (row_index * width) % 4 if vec else np.zeros(n, dtype=np.int64)
    for shift in range(4):
        sel = np.nonzero(shifts == shift)[0]
        if len(sel) == 0:
            continue
        part = sq[sel]
        ys = []
        for y in range(bh):
            v = [_thread_sum(part, width, x_, y, sched, shift) for x_ in range(bw)]
            off = bw // 2
            while off >= 64:  # block_x_reduce through shared memory
                for t in range(off):
                    v[t] = (v[t] + v[t + off]).astype(_F32)
                off //= 2
            dim, off = min(bw, 64), 1
            while off < dim:  # then v += shfl_down(v, off), off = 1, 2, 4, ...
                for t in range(dim - off):
                    v[t] = (v[t] + v[t + off]).astype(_F32)
                off *= 2
            ys.append(v[0])
        off = bh // 2
        while off > 0:  # block_y_reduce
            for y in range(off):
                ys[y] = (ys[y] + ys[y + off]).astype(_F32)
            off //= 2
        out[sel] = ys[0]
    return out


def device_rstd(row_sums: np.ndarray, rows: int, width: int, eps: float) -> np.ndarray:
    """MeanOps' projection (sum * float(rows) / numel), + eps in fp32, then the
    correctly rounded reciprocal square root (torch.rsqrt on the GPU)."""
    factor = _F32(_F32(rows) / _F32(rows * width))
    var = (row_sums.astype(_F32) * factor).astype(_F32)
    v = (var + _F32(eps)).astype(_F32)
    with np.errstate(divide="ignore", invalid="ignore"):
        return (1.0 / np.sqrt(v.astype(np.float64))).astype(_F32)


def device_forward(hidden: torch.Tensor, weight: torch.Tensor, eps: float):
    """The stock forward's bytes on the GPU: (primal, rstd[..., 1] fp32).

    Same operations as :func:`rms_norm_forward`; only the variance's summation
    order and the rsqrt rounding are the GPU's.
    """
    width = hidden.shape[-1]
    x = hidden.detach().float().reshape(-1, width).numpy()
    rows = x.shape[0]
    r = device_rstd(device_row_sums(x), rows, width, eps)
    rstd = torch.from_numpy(r).reshape(*hidden.shape[:-1], 1)
    xhat = (hidden.detach().float() * rstd).to(hidden.dtype)
    return weight.detach() * xhat, rstd
