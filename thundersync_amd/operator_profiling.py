"""Named ranges around the operators, off unless asked for.

Interface of the reference's ``accel/operator_profiling.py`` (names,
``THUNDERSYNC_OPERATOR_PROFILE_RANGES``, modes, the range-name format
``thundersync::<category>|key=value|...``), built for ROCm:

* a mode is a pair of switches -- profiler ranges (``kineto``: a torch
  ``record_function`` that the torch profiler shows) and ROCTx markers
  (``roctx``, which ``rocprofv3 --marker-trace`` records; ``nvtx`` is taken
  as its name in configurations written for the reference) -- ``both`` sets
  both, ``off`` neither;
* markers go straight to the ROCTx library through ctypes
  (``roctxRangePushA`` / ``roctxRangePop``, thread-local stacks), with
  torch's marker wrapper only where no ROCTx library loads;
* a range is a small object with ``__enter__`` / ``__exit__``; with
  profiling off :func:`operator_range` returns one shared do-nothing
  instance, so a disabled range costs one global read and no torch or HIP
  call.
"""

from __future__ import annotations

import ctypes
import os
import threading
from collections.abc import Mapping

import torch

PROFILE_RANGES_ENV = "THUNDERSYNC_OPERATOR_PROFILE_RANGES"

# mode -> (profiler ranges, ROCTx markers)
_SWITCHES = {"off": (False, False), "kineto": (True, False), "roctx": (False, True), "both": (True, True)}
_SYNONYMS = {"nvtx": "roctx"}


class _State:
    mode: str | None = None  # None until first use reads the environment
    roles: dict[str, str] = {}


def _parse(text: str, where: str) -> str:
    name = _SYNONYMS.get(text.strip().lower(), text.strip().lower())
    if name not in _SWITCHES:
        raise ValueError(f"{where}: {text!r} is not one of {', '.join([*_SWITCHES, *_SYNONYMS])}")
    return name


def _mode() -> str:
    if _State.mode is None:
        _State.mode = _parse(os.environ.get(PROFILE_RANGES_ENV, "off"), PROFILE_RANGES_ENV)
    return _State.mode


def configure_operator_profiling(mode: str, *, device_roles: Mapping[str, str] | None = None) -> None:
    """Set the process-wide mode (and names for devices, e.g. teacher/student)."""
    _State.mode = _parse(mode, "operator profiling mode")
    _State.roles = {str(torch.device(d)): str(role) for d, role in (device_roles or {}).items()}


def operator_profiling_mode() -> str:
    return _mode()


def operator_profiling_enabled() -> bool:
    return _mode() != "off"


def device_role(device) -> str:
    """The configured role name of a device, else the device's own name."""
    key = str(torch.device(device))
    return _State.roles.get(key, key)


def range_name(category: str, **fields: object) -> str:
    """``thundersync::<category>|key=value|...``; values lose ``|`` and newlines."""
    name = "thundersync::" + category
    for key, value in fields.items():
        if value is not None:
            name += f"|{key}=" + str(value).translate(_CLEAN)
    return name


_CLEAN = str.maketrans({"|": "/", "\n": " "})


class _Markers:
    """ROCTx push/pop, resolved once."""

    _lock = threading.Lock()
    _api: tuple | None = None

    @classmethod
    def api(cls):
        if cls._api is None:
            with cls._lock:
                if cls._api is None:
                    cls._api = cls._load()
        return cls._api

    @staticmethod
    def _load():
        for lib in ("librocprofiler-sdk-roctx.so.1", "libroctx64.so.4", "/opt/rocm/lib/libroctx64.so"):
            try:
                handle = ctypes.CDLL(lib)
                push, pop = handle.roctxRangePushA, handle.roctxRangePop
            except (OSError, AttributeError):
                continue
            push.argtypes, push.restype = [ctypes.c_char_p], ctypes.c_int
            pop.argtypes, pop.restype = [], ctypes.c_int
            return (lambda name: push(name.encode()), pop)
        return (torch.cuda.nvtx.range_push, torch.cuda.nvtx.range_pop)


class _Range:
    __slots__ = ("name", "kineto", "marker", "_record")

    def __init__(self, name: str, kineto: bool, marker: bool):
        self.name, self.kineto, self.marker, self._record = name, kineto, marker, None

    def __enter__(self):
        if self.kineto:
            self._record = torch.profiler.record_function(self.name)
            self._record.__enter__()
        if self.marker:
            _Markers.api()[0](self.name)
        return None

    def __exit__(self, *exc):
        if self.marker:
            _Markers.api()[1]()
        if self._record is not None:
            self._record.__exit__(None, None, None)
            self._record = None
        return False


class _Nothing:
    __slots__ = ()

    def __enter__(self):
        return None

    def __exit__(self, *exc):
        return False


_NOTHING = _Nothing()


def operator_range(category: str, *, fields: Mapping[str, object] | None = None, **named: object):
    """A context manager around one operator: the shared do-nothing range when
    profiling is off, else a range named by :func:`range_name`."""
    mode = _State.mode if _State.mode is not None else _mode()
    if mode == "off":
        return _NOTHING
    kineto, marker = _SWITCHES[mode]
    return _Range(range_name(category, **{**(fields or {}), **named}), kineto, marker)
