"""Trial-once availability of a kernel on a device.

Contract of the reference's ``accel/capability.py:61-129``: a kernel is tried
once per ``(kernel, device index, dtype, shape key)`` with gradients enabled
and the device synchronized; the outcome (and the error text of a failure) is
cached and reported by :func:`kernel_probe_records`.  A CPU tensor never runs
a device kernel.  The trial never wraps a real call, so a real failure still
raises where it happens.
"""

from __future__ import annotations

import threading
from collections.abc import Callable
from typing import NamedTuple

import torch

__all__ = ["device_identity", "kernel_probe_records", "kernel_runs", "reset_kernel_probes"]


class _Outcome(NamedTuple):
    runs: bool
    error: str | None


_GUARD = threading.Lock()
_CACHE: dict[tuple[str, int, str, int], _Outcome] = {}


def device_identity(device: torch.device | int | None = None) -> dict[str, object]:
    """Name, architecture and memory of a GPU, or ``{}`` without one."""
    if not torch.cuda.is_available():
        return {}
    if isinstance(device, int):
        index = device
    elif device is not None and getattr(device, "index", None) is not None:
        index = device.index
    else:
        index = torch.cuda.current_device()
    props = torch.cuda.get_device_properties(index)
    return {
        "index": index,
        "name": props.name,
        "arch": getattr(props, "gcnArchName", ""),
        "compute_capability": f"{props.major}.{props.minor}",
        "total_memory_mib": props.total_memory // (1 << 20),
        "multiprocessors": props.multi_processor_count,
    }


def kernel_runs(
    kernel: str,
    like,
    shape_key: int,
    trial: Callable[[torch.device, torch.dtype, int], None],
) -> bool:
    """Whether ``trial`` completes on ``like``'s device and dtype (cached)."""
    if not like.is_cuda:
        return False
    key = (kernel, like.device.index, str(like.dtype), shape_key)
    hit = _CACHE.get(key)
    if hit is not None:
        return hit.runs
    with _GUARD:
        hit = _CACHE.get(key)
        if hit is None:
            hit = _attempt(trial, like.device, like.dtype, shape_key)
            _CACHE[key] = hit
    return hit.runs


def _attempt(trial, device, dtype, shape_key) -> _Outcome:
    try:
        with torch.cuda.device(device), torch.enable_grad():
            trial(device, dtype, shape_key)
            torch.cuda.synchronize(device)
    except Exception as error:  # any failure means "does not run here"
        return _Outcome(False, f"{type(error).__name__}: {str(error)[:300]}")
    return _Outcome(True, None)


def kernel_probe_records() -> list[dict[str, object]]:
    """Every trial this process ran, with the device it ran on."""
    seen: dict[int, dict[str, object]] = {}
    out = []
    for (kernel, index, dtype, shape_key), outcome in sorted(_CACHE.items()):
        if index not in seen:
            seen[index] = device_identity(index)
        out.append(
            {
                "kernel": kernel,
                "device": seen[index],
                "dtype": dtype,
                "shape_key": shape_key,
                "runs": outcome.runs,
                "error": outcome.error,
            }
        )
    return out


def reset_kernel_probes() -> None:
    """Forget every outcome (tests re-probe with it)."""
    with _GUARD:
        _CACHE.clear()
