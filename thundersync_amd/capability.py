"""Whether a kernel runs on a device, decided once by running it.

The reference decides this per ``(kernel, device index, dtype, shape key)``
by a small trial with gradients enabled, the device synchronized afterwards
so that an asynchronous launch failure surfaces inside the trial, and the
outcome cached for the process (accel/capability.py:61-129).  The public
names, signatures and record keys below are that contract; the machinery
is this module's own:

* every key owns a :class:`_Probe` whose ``threading.Event`` marks the
  outcome as known, so two keys (two devices of a teacher/student pair, two
  dtypes) probe concurrently and a caller racing a running trial of the same
  key waits for it instead of running it twice;
* a probe records the trial's wall time and the device it ran on, taken when
  the trial ran.

A CPU tensor never runs a device kernel, and a trial never wraps a real
call: a real failure still raises where it happens.
"""

from __future__ import annotations

import threading
import time
import traceback
from collections.abc import Callable
from dataclasses import dataclass, field

import torch

__all__ = ["device_identity", "kernel_probe_records", "kernel_runs", "reset_kernel_probes"]

Trial = Callable[[torch.device, torch.dtype, int], None]
_ERROR_CHARS = 300


def device_identity(device: torch.device | int | None = None) -> dict[str, object]:
    """What a GPU is: index, name, architecture, memory; ``{}`` without a GPU."""
    if not torch.cuda.is_available():
        return {}
    index = device if isinstance(device, int) else getattr(device, "index", None)
    if index is None:
        index = torch.cuda.current_device()
    p = torch.cuda.get_device_properties(index)
    return {
        "index": index,
        "name": p.name,
        "arch": getattr(p, "gcnArchName", ""),
        "compute_capability": f"{p.major}.{p.minor}",
        "total_memory_mib": p.total_memory >> 20,
        "multiprocessors": p.multi_processor_count,
    }


@dataclass
class _Probe:
    """One key's trial: run at most once, outcome published through `done`."""

    done: threading.Event = field(default_factory=threading.Event)
    claimed: bool = False
    runs: bool = False
    error: str | None = None
    seconds: float = 0.0
    device: dict[str, object] = field(default_factory=dict)

    def run(self, trial: Trial, device: torch.device, dtype: torch.dtype, shape_key: int) -> None:
        start = time.perf_counter()
        try:
            with torch.cuda.device(device):
                with torch.enable_grad():
                    trial(device, dtype, shape_key)
                torch.cuda.synchronize(device)
            self.runs = True
        except Exception as failure:  # any failure means: not on this device
            text = "".join(traceback.format_exception_only(type(failure), failure)).strip()
            self.runs, self.error = False, text[:_ERROR_CHARS]
        self.seconds = time.perf_counter() - start
        self.device = device_identity(device)
        self.done.set()


class _Registry:
    def __init__(self) -> None:
        self._guard = threading.Lock()
        self._probes: dict[tuple[str, int, str, int], _Probe] = {}

    def outcome(self, key, trial: Trial, device: torch.device, dtype: torch.dtype, shape_key: int) -> bool:
        with self._guard:
            probe = self._probes.setdefault(key, _Probe())
            mine = not probe.claimed
            probe.claimed = True
        if mine:
            probe.run(trial, device, dtype, shape_key)
        else:
            probe.done.wait()
        return probe.runs

    def records(self) -> list[dict[str, object]]:
        with self._guard:
            items = sorted((k, p) for k, p in self._probes.items() if p.done.is_set())
        return [
            {"kernel": k[0], "device": p.device, "dtype": k[2], "shape_key": k[3], "runs": p.runs,
             "error": p.error, "seconds": round(p.seconds, 6)}
            for k, p in items
        ]

    def clear(self) -> None:
        with self._guard:
            self._probes = {k: p for k, p in self._probes.items() if not p.done.is_set()}


_REGISTRY = _Registry()


def kernel_runs(kernel: str, like: torch.Tensor, shape_key: int, trial: Trial) -> bool:
    """Whether ``trial(device, dtype, shape_key)`` completes on ``like``'s device
    and dtype; the trial runs at most once per key in this process."""
    if not like.is_cuda:
        return False
    key = (kernel, like.device.index, str(like.dtype), int(shape_key))
    return _REGISTRY.outcome(key, trial, like.device, like.dtype, int(shape_key))


def kernel_probe_records() -> list[dict[str, object]]:
    """One record per finished trial: kernel, device, dtype, shape_key, runs,
    error (None when it ran) and the trial's wall time in seconds."""
    return _REGISTRY.records()


def reset_kernel_probes() -> None:
    """Forget finished outcomes (a trial still running keeps its entry)."""
    _REGISTRY.clear()
