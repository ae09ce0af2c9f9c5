"""Loading libthundersync_hip.so and the ``THUNDERSYNC_HIP`` switch.

The switch has the semantics of the reference's ``THUNDERSYNC_FA4``
(src/thundersync/engine/streaming.py:395-505):

* ``require`` -- every resolution that cannot load the library raises, and
  the failure is not cached, so every later dispatch raises again;
* ``off`` -- the library is never loaded; the resolution returns None;
* ``auto`` (also the value when the variable is unset) -- the library is
  loaded when it can be; otherwise the resolution returns None.

The resolution happens once, under a lock, and is cached until
:func:`reset` clears it.  :func:`library` is what the integration point (the
reference's attention dispatch, or a test) consults; the operators in this
package call :func:`require_library`, which raises whenever the library is
not available -- there is no host fallback inside this package.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

from ._abi import AttnProblem, AttnRows

HIP_ENV = "THUNDERSYNC_HIP"
HIP_SETTINGS = ("require", "off", "auto")
LIB_NAME = "libthundersync_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

# Every symbol include/thundersync_hip.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F = ctypes.c_float
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ts_hip_version": (ctypes.c_char_p, []),
    "ts_hip_last_error": (ctypes.c_char_p, []),
    "ts_rmsnorm_fwd": (_INT, [_P, _P, _P, _P, _I64, _I64, _F, _INT, _P]),
    "ts_rmsnorm_supported": (_INT, [_I64, _I64, _P]),
    "ts_rmsnorm_bwd_workspace": (_I64, [_I64, _I64]),
    "ts_rmsnorm_bwd": (_INT, [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _INT, _P]),
    "ts_rmsnorm_bwd_noalloc": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _P]),
    "ts_device_clocks": (_INT, [_INT, ctypes.POINTER(_INT), ctypes.POINTER(_INT), ctypes.POINTER(_INT),
                                ctypes.POINTER(_INT)]),
    "ts_timing_enable": (_INT, [_INT]),
    "ts_timing_reset": (_INT, []),
    "ts_timing_read": (_INT, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_I64)]),
    "ts_logprob_fwd_workspace": (_I64, [_I64, _I64]),
    "ts_logprob_fwd": (_INT, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _INT, _P]),
    "ts_logprob_dlogits": (
        _INT,
        [_P, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _INT, _P],
    ),
    "ts_logprob_grad_hidden_workspace": (_I64, [_I64, _I64, _I64]),
    "ts_logprob_grad_hidden": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64, _INT, _P]),
    "ts_logprob_grad_weight": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _INT, _P]),
    "ts_logprob_fwd_exact_workspace": (_I64, [_I64, _I64, _INT]),
    "ts_logprob_fwd_exact": (_INT, [_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _INT, _P]),
    "ts_logprob_dlogits_exact": (
        _INT,
        [_P, _I64, _P, _I64, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _I64, _INT, _P],
    ),
    "ts_matmul_exact": (_INT, [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _INT, _INT, _P]),
    "ts_lora_fwd": (_INT, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _INT, _P]),
    "ts_lora_bwd_workspace": (_I64, [_I64, _I64, _I64, _I64]),
    "ts_lora_bwd": (
        _INT,
        [_P, _I64, _P, _I64, _P, _I64, _P, _P, _I64, ctypes.c_float, _I64, _I64, _I64, _P, _I64, _P, _P, _P, _I64,
         _INT, _P],
    ),
    "ts_adjoint_reduce": (_INT, [ctypes.POINTER(_P), _INT, _P, _P, _I64, _INT, _P]),
    "ts_ledger_add": (_INT, [_P, _P, _I64, _INT, _INT, _P]),
    "ts_forest_build": (_INT, [_I64, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _P]),
    "ts_plan_compile": (_INT, [_I64, _P, _P, _P, _P, _P, _I64, _P, _P, _I64] + [_P] * 13),
    "ts_attn_heads_per_block": (_INT, [_INT]),
    "ts_attn_kv_block": (_INT, [_INT, _INT]),
    "ts_attn_q_block": (_INT, [_INT]),
    "ts_attn_check_tables": (_INT, [ctypes.POINTER(AttnProblem), _P, _P, _I64, _P, _P, _I64, _P, _P]),
    "ts_attn_fwd": (_INT, [ctypes.POINTER(AttnProblem), AttnRows, AttnRows, _P, _I64, _P]),
    "ts_attn_bwd": (
        _INT,
        [ctypes.POINTER(AttnProblem), AttnRows, AttnRows, AttnRows, _P, _I64, _P, AttnRows, _P],
    ),
    "ts_attn_ds_route": (_INT, [_INT, _INT]),
    "ts_attn_ds_layout": (
        _INT,
        [_P, ctypes.c_int32, _P, _I64, _P, ctypes.c_int32, _P, _P, _P, _I64, _P, _P, ctypes.POINTER(_I64)],
    ),
    "ts_attn_bwd_ds": (
        _INT,
        [ctypes.POINTER(AttnProblem), AttnRows, AttnRows, AttnRows, _P, _I64, _P, AttnRows, _P, _P, _I64, _P,
         _I64, _P, ctypes.c_int32, ctypes.c_int32, _P],
    ),
}

TS_OK = 0
TS_F32, TS_F16, TS_BF16, TS_F64 = 0, 1, 2, 3

_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None
_RESOLVED = False
_SETTING: str | None = None


def hip_setting() -> str:
    """The ``THUNDERSYNC_HIP`` setting: ``require``, ``off`` or ``auto``."""
    value = os.environ.get(HIP_ENV, "auto").strip().lower() or "auto"
    if value not in HIP_SETTINGS:
        raise ValueError(f"{HIP_ENV} must be one of {', '.join(HIP_SETTINGS)}, not {value!r}")
    return value


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise OSError(f"{LIB_PATH} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def library() -> ctypes.CDLL | None:
    """The library, resolved once under ``THUNDERSYNC_HIP``, or None."""
    global _LIB, _RESOLVED, _SETTING
    if _RESOLVED:
        return _LIB
    with _LOCK:
        if _RESOLVED:
            return _LIB
        setting = hip_setting()
        if setting == "off":
            _LIB, _SETTING, _RESOLVED = None, setting, True
            return None
        try:
            lib = _load()
        except Exception as error:
            if setting == "require":
                raise RuntimeError(
                    f"{HIP_ENV}=require but {LIB_NAME} cannot be loaded: {error!r}"
                ) from error
            lib = None
        _LIB, _SETTING, _RESOLVED = lib, setting, True
        return lib


def resolved_setting() -> str | None:
    """The setting the last completed resolution read, or None before one."""
    return _SETTING


def hip_build() -> str | None:
    """Diagnostic: the loaded library's version string, or None. Never raises."""
    try:
        lib = library()
    except RuntimeError:
        return None
    return None if lib is None else lib.ts_hip_version().decode()


def reset() -> None:
    """Forget the resolution; the next call re-reads the setting."""
    global _LIB, _RESOLVED, _SETTING
    with _LOCK:
        _LIB, _RESOLVED, _SETTING = None, False, None


def require_library() -> ctypes.CDLL:
    """The library, or an error that says why it is not available."""
    lib = library()
    if lib is None:
        if _SETTING == "off":
            raise RuntimeError(f"the HIP kernels are switched off ({HIP_ENV}=off)")
        raise RuntimeError(
            f"{LIB_NAME} is not available; build it with __graft_entry__.build()"
        )
    return lib


def check(status: int, what) -> None:
    """Raise RuntimeError naming the kernel call when a status is not TS_OK;
    ``what`` is the call's description, or a function that builds it (so a
    hot call site formats nothing when the call succeeds)."""
    if status != TS_OK:
        lib = require_library()
        message = lib.ts_hip_last_error().decode()
        if callable(what):
            what = what()
        raise RuntimeError(f"{what} failed (status {status}): {message}")


_DTYPE_CODES: dict | None = None


def dtype_code(dtype) -> int:
    global _DTYPE_CODES
    if _DTYPE_CODES is None:
        import torch

        _DTYPE_CODES = {torch.float32: TS_F32, torch.float16: TS_F16, torch.bfloat16: TS_BF16,
                        torch.float64: TS_F64}
    code = _DTYPE_CODES.get(dtype)
    if code is None:
        raise TypeError(f"unsupported dtype {dtype}")
    return code


def stream_of(tensor) -> int:
    """The current HIP stream of ``tensor``'s device, as an integer handle."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None and tensor.device.index is not None:
        return raw(tensor.device.index)
    return torch.cuda.current_stream(tensor.device).cuda_stream


def ptr(tensor) -> int | None:
    return None if tensor is None else tensor.data_ptr()


def device_clocks(device: int = 0) -> dict[str, int]:
    """Compute units, peak engine clock, memory clock (kHz) and memory bus
    width (bits) of a device, from hipDeviceGetAttribute (ts_device_clocks)."""
    lib = require_library()
    vals = [ctypes.c_int() for _ in range(4)]
    check(lib.ts_device_clocks(int(device), *(ctypes.byref(v) for v in vals)), "ts_device_clocks")
    return dict(zip(("cus", "clock_khz", "mem_clock_khz", "mem_bus_bits"), (v.value for v in vals)))


class KernelTimer:
    """Per-kernel device time of the library's launches inside a ``with`` block.

    Uses the library's HIP-event brackets (ts_timing_*), which are recorded
    on the stream each kernel is launched on.
    """

    def __enter__(self):
        lib = require_library()
        lib.ts_timing_reset()
        lib.ts_timing_enable(1)
        return self

    def __exit__(self, *exc):
        require_library().ts_timing_enable(0)
        return False

    @staticmethod
    def read(kernel: str) -> tuple[float, int]:
        """(total milliseconds, launches) of ``kernel`` since the last reset."""
        lib = require_library()
        total = ctypes.c_double()
        n = ctypes.c_int64()
        check(lib.ts_timing_read(kernel.encode(), ctypes.byref(total), ctypes.byref(n)), "ts_timing_read")
        return total.value, n.value
