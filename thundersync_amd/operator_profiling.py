"""Disabled-by-default named ranges around the operators.

Same contract as the reference's ``accel/operator_profiling.py:1-161``: the
mode is ``off`` (default), ``kineto``, ``roctx`` or ``both``, read lazily
from ``THUNDERSYNC_OPERATOR_PROFILE_RANGES`` or set by
:func:`configure_operator_profiling`; range names have the stable form
``thundersync::<category>|key=value|...``.  With profiling off, entering a
range makes no torch or HIP call.  On ROCm the marker API is roctx; torch
exposes it through ``torch.cuda.nvtx``, so ``nvtx`` is accepted as an alias
of ``roctx`` for configurations written for the reference.
"""

from __future__ import annotations

import os
from collections.abc import Iterator, Mapping
from contextlib import contextmanager

import torch

PROFILE_RANGES_ENV = "THUNDERSYNC_OPERATOR_PROFILE_RANGES"
_MODES = ("off", "kineto", "roctx", "both")
_ALIASES = {"nvtx": "roctx"}
_mode: str | None = None
_roles: dict[str, str] = {}


def _normalize(mode: str, source: str) -> str:
    value = mode.strip().lower()
    value = _ALIASES.get(value, value)
    if value not in _MODES:
        raise ValueError(f"{source} must be one of {sorted(_MODES)} (or nvtx), got {mode!r}")
    return value


def _current() -> str:
    global _mode
    if _mode is None:
        _mode = _normalize(os.environ.get(PROFILE_RANGES_ENV, "off"), PROFILE_RANGES_ENV)
    return _mode


def configure_operator_profiling(mode: str, *, device_roles: Mapping[str, str] | None = None) -> None:
    """Set the process-wide range mode and optional device role names."""
    global _mode, _roles
    _mode = _normalize(mode, "operator profiling mode")
    _roles = {str(torch.device(d)): str(r) for d, r in (device_roles or {}).items()}


def operator_profiling_mode() -> str:
    return _current()


def operator_profiling_enabled() -> bool:
    return _current() != "off"


def device_role(device) -> str:
    name = str(torch.device(device))
    return _roles.get(name, name)


def range_name(category: str, **fields: object) -> str:
    parts = [f"thundersync::{category}"]
    for key, value in fields.items():
        if value is not None:
            parts.append(f"{key}={str(value).replace('|', '/').replace(chr(10), ' ')}")
    return "|".join(parts)


class _Off:
    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_OFF = _Off()


@contextmanager
def _on(mode: str, category: str, fields: Mapping[str, object]) -> Iterator[None]:
    name = range_name(category, **fields)
    record = torch.profiler.record_function(name) if mode in ("kineto", "both") else None
    marker = mode in ("roctx", "both")
    if record is not None:
        record.__enter__()
    pushed = False
    try:
        if marker:
            torch.cuda.nvtx.range_push(name)
            pushed = True
        yield
    finally:
        if pushed:
            torch.cuda.nvtx.range_pop()
        if record is not None:
            record.__exit__(None, None, None)


def operator_range(category: str, *, fields: Mapping[str, object] | None = None, **named: object):
    """A no-op singleton when off, else a range named ``thundersync::category|...``."""
    mode = _mode if _mode is not None else _current()
    if mode == "off":
        return _OFF
    merged = dict(fields or {})
    merged.update(named)
    return _on(mode, category, merged)
