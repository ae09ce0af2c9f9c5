"""Whether a call may take the HIP kernels, and which path served each call.

The integration point of the reference's attention dispatch
(engine/streaming.py:355-373, :414-548) for this library:

* :func:`hip_attention_available` / :func:`hip_logprob_available` answer for
  one call's tensors.  Under ``THUNDERSYNC_HIP=off`` (or ``auto`` without a
  loadable library) the answer is no; under ``require`` a library that cannot
  load raises at every call (``_lib.library``), and a loaded one is used
  without a trial, so that a kernel that cannot run on the device fails at
  the call instead of falling through; under ``auto`` the kernels are taken
  once a trial -- forward and backward of a tiny problem, once per
  ``(device, dtype, head_dim)`` -- has run on that device
  (:func:`thundersync_amd.capability.kernel_runs`).
* :func:`count_attention_path` / :func:`attention_path_counts` record, per
  path name, how many attention calls it served (the operators count
  ``hip`` per forward launch and ``hip_backward`` per backward launch).

The operators themselves never consult this module: they always run the
kernels and raise when they cannot; choosing another path is the caller's.
"""

from __future__ import annotations

import threading
from collections import Counter

import torch

from . import _lib
from .capability import kernel_runs

HIP_PATH = "hip"
HIP_BACKWARD_PATH = "hip_backward"

_counts: Counter[str] = Counter()
_counts_lock = threading.Lock()


def count_attention_path(name: str, calls: int = 1) -> None:
    """Record ``calls`` attention calls served by path ``name``."""
    with _counts_lock:
        _counts[name] += calls


def attention_path_counts() -> dict[str, int]:
    """Attention calls served per path in this process, cumulative, by name."""
    with _counts_lock:
        return dict(sorted(_counts.items()))


def reset_attention_path_counts() -> None:
    with _counts_lock:
        _counts.clear()


def attention_trial(device: torch.device, dtype: torch.dtype, head_dim: int) -> None:
    """Eight queries over a 16-key bottom-right window, 4 query heads on one KV
    head: the forward and every input gradient, finite."""
    from .attention import causal_attention

    g = torch.Generator(device=device).manual_seed(0)

    def leaf(*shape):
        return torch.randn(*shape, device=device, dtype=dtype, generator=g).requires_grad_()

    q, k, v = leaf(1, 4, 8, head_dim), leaf(16, 1, head_dim), leaf(16, 1, head_dim)
    out = causal_attention(q, [k], [v], head_dim ** -0.5)
    grads = torch.autograd.grad(out.float().square().sum(), (q, k, v))
    if not all(bool(t.isfinite().all()) for t in (out, *grads)):
        raise RuntimeError("HIP attention trial produced nonfinite values")


def logprob_trial(device: torch.device, dtype: torch.dtype, dim: int) -> None:
    """Five rows over a 300-token head: logprob, entropy and the hidden gradient, finite."""
    from .fused_logprob import fused_logprob_entropy

    g = torch.Generator(device=device).manual_seed(0)
    h = torch.randn(5, dim, device=device, dtype=dtype, generator=g).requires_grad_()
    w = torch.randn(300, dim, device=device, dtype=dtype, generator=g) * 0.02
    t = torch.randint(0, 300, (5,), device=device, generator=g)
    lp, ent = fused_logprob_entropy(h, w, t, chunk=4)
    (grad,) = torch.autograd.grad((lp + ent).sum(), (h,))
    if not all(bool(x.isfinite().all()) for x in (lp, ent, grad)):
        raise RuntimeError("HIP logprob trial produced nonfinite values")


def _available(like: torch.Tensor, kernel: str, key: int, trial,
               dtypes=(torch.bfloat16, torch.float16)) -> bool:
    if not like.is_cuda or like.dtype not in dtypes:
        return False
    if _lib.library() is None:  # off, or auto without a library; require raises
        return False
    if _lib.resolved_setting() == "require":
        return True
    return kernel_runs(kernel, like, key, trial)


def hip_attention_available(query: torch.Tensor) -> bool:
    """Whether this query (any layout with the head dim last) may take the HIP attention."""
    from .attention import kernel_head_dim

    if kernel_head_dim(int(query.shape[-1])) is None:
        return False
    return _available(query, "hip_attention", int(query.shape[-1]), attention_trial)


def hip_logprob_available(hidden: torch.Tensor) -> bool:
    """Whether these hidden states may take the HIP fused logprob (bf16 and
    fp16 on MFMA; fp32 and fp64 at their own precision)."""
    return _available(hidden, "hip_logprob", int(hidden.shape[-1]), logprob_trial,
                      (torch.bfloat16, torch.float16, torch.float32, torch.float64))
