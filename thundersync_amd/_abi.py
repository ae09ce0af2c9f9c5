"""ctypes / numpy mirrors of the C structures in include/thundersync_hip.h."""

from __future__ import annotations

import ctypes

import numpy as np

SEG_DTYPE = np.dtype(
    [("q_row0", "<i8"), ("q_len", "<i4"), ("kv_len", "<i4"), ("span0", "<i4"), ("nspan", "<i4")]
)
REF_DTYPE = np.dtype([("index", "<i4"), ("kpos", "<i4")])
RUN_DTYPE = np.dtype(
    [
        ("k", "<u8"), ("v", "<u8"), ("dk", "<u8"), ("dv", "<u8"),
        ("k_row_stride", "<i8"), ("k_head_stride", "<i8"),
        ("v_row_stride", "<i8"), ("v_head_stride", "<i8"),
        ("dk_row_stride", "<i8"), ("dk_head_stride", "<i8"),
        ("dv_row_stride", "<i8"), ("dv_head_stride", "<i8"),
        ("len", "<i4"), ("visit0", "<i4"), ("nvisit", "<i4"), ("reserved", "<i4"),
    ]
)


class AttnProblem(ctypes.Structure):
    """ts_attn_problem"""

    _fields_ = [
        ("segs", ctypes.c_void_p),
        ("seg_spans", ctypes.c_void_p),
        ("runs", ctypes.c_void_p),
        ("run_visits", ctypes.c_void_p),
        ("q_work", ctypes.c_void_p),
        ("kv_work", ctypes.c_void_p),
        ("n_q_work", ctypes.c_int32),
        ("n_kv_work", ctypes.c_int32),
        ("n_segs", ctypes.c_int32),
        ("n_runs", ctypes.c_int32),
        ("hq", ctypes.c_int32),
        ("hkv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("q_block", ctypes.c_int32),
        ("kv_block", ctypes.c_int32),
        ("q_rows", ctypes.c_int64),
        ("n_q_long", ctypes.c_int32),
        ("n_kv_long", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


class AttnRows(ctypes.Structure):
    """ts_attn_rows"""

    _fields_ = [("ptr", ctypes.c_uint64), ("row_stride", ctypes.c_int64), ("head_stride", ctypes.c_int64)]


assert SEG_DTYPE.itemsize == 24 and REF_DTYPE.itemsize == 8 and RUN_DTYPE.itemsize == 112
assert ctypes.sizeof(AttnProblem) == 112 and ctypes.sizeof(AttnRows) == 24
