"""Pin the MFMA and register-transpose lane layouts the kernels assume.

One wave runs v_mfma_f32_16x16x32_bf16, v_mfma_f32_32x32x16_bf16 and the
8x8 16-bit register transpose on integer-valued bf16 operands (exact in
fp32), and the result is compared with the layouts written in
thundersync_amd/csrc/common.h, computed here with numpy.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.probe.build_probe import LIB_PATH as PROBE_LIB
from thundersync_amd import _lib

pytestmark = pytest.mark.gpu

_P, _INT = ctypes.c_void_p, ctypes.c_int
PROBE_SIGNATURES = {
    "ts_probe_last_error": (ctypes.c_char_p, []),
    "ts_probe_layouts": (_INT, [_P] * 7),
    "ts_probe_lds": (_INT, [_P] * 5 + [_INT, _P]),
    "ts_probe_lanes": (_INT, [_P] * 3),
    "ts_probe_dma_offset": (_INT, [_P] * 3),
}


def probe_library() -> ctypes.CDLL:
    """The test-only probe library (tests/probe/libts_probe.so)."""
    if not PROBE_LIB.exists():
        pytest.fail(f"{PROBE_LIB} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(PROBE_LIB))
    for name, (restype, argtypes) in PROBE_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = restype, argtypes
    return lib


def probe_check(lib, status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"{what} failed (status {status}): {lib.ts_probe_last_error().decode()}")


def expected_16(a, b):
    # a, b: [64 lanes, 8 slots]; A[row=l%16][k=8*(l//16)+j], B[k][col=l%16]
    A = np.zeros((16, 32))
    B = np.zeros((32, 16))
    for l in range(64):
        for j in range(8):
            A[l % 16, 8 * (l // 16) + j] = a[l, j]
            B[8 * (l // 16) + j, l % 16] = b[l, j]
    D = A @ B
    out = np.zeros((64, 4))
    for l in range(64):
        for i in range(4):
            out[l, i] = D[4 * (l // 16) + i, l % 16]
    return out


def expected_32(a, b):
    A = np.zeros((32, 16))
    B = np.zeros((16, 32))
    for l in range(64):
        for j in range(8):
            A[l % 32, 8 * (l // 32) + j] = a[l, j]
            B[8 * (l // 32) + j, l % 32] = b[l, j]
    D = A @ B
    out = np.zeros((64, 16))
    for l in range(64):
        for i in range(16):
            out[l, i] = D[8 * (i // 4) + 4 * (l // 32) + (i % 4), l % 32]
    return out


def test_mfma_and_transpose_layouts(cuda):
    lib = probe_library()
    rng = np.random.default_rng(0)
    a = rng.integers(-4, 5, size=(64, 8)).astype(np.float32)
    b = rng.integers(-4, 5, size=(64, 8)).astype(np.float32)
    t_in = rng.integers(-100, 100, size=(64, 8, 8)).astype(np.float32)
    da = torch.tensor(a, dtype=torch.bfloat16, device=cuda)
    db = torch.tensor(b, dtype=torch.bfloat16, device=cuda)
    dt = torch.tensor(t_in, dtype=torch.bfloat16, device=cuda)
    d16 = torch.empty(64, 4, dtype=torch.float32, device=cuda)
    d32 = torch.empty(64, 16, dtype=torch.float32, device=cuda)
    t_out = torch.empty(64, 8, 8, dtype=torch.bfloat16, device=cuda)
    print("probe: ts_probe_layouts", flush=True)
    probe_check(
        lib,
        lib.ts_probe_layouts(da.data_ptr(), db.data_ptr(), d16.data_ptr(), d32.data_ptr(),
                             dt.data_ptr(), t_out.data_ptr(), _lib.stream_of(da)),
        "ts_probe_layouts",
    )
    torch.cuda.synchronize()
    np.testing.assert_array_equal(d16.cpu().numpy(), expected_16(a, b))
    np.testing.assert_array_equal(d32.cpu().numpy(), expected_32(a, b))
    np.testing.assert_array_equal(
        t_out.float().cpu().numpy(), np.transpose(t_in, (0, 2, 1))
    )


def test_lds_dma_and_transpose_read_layouts(cuda):
    """Record where global_load_lds_dwordx4 puts each lane's 16 bytes, and the
    lane mapping of ds_read_b64_tr_b16 over contiguous 8-byte rows."""
    lib = probe_library()
    src = torch.arange(64 * 4, dtype=torch.int32, device=cuda)  # 16 bytes per lane: 4l..4l+3
    perm = torch.tensor(np.random.default_rng(1).permutation(64), dtype=torch.int32, device=cuda)
    dma = torch.empty(64 * 4, dtype=torch.int32, device=cuda)
    tr = torch.empty(64 * 4, dtype=torch.int16, device=cuda)
    buf = torch.empty(64 * 4, dtype=torch.int32, device=cuda)
    valid = 16 * 37 + 8  # rows 0..36 in range; row 37 straddles the end; 38.. out of range
    print("probe: ts_probe_lds", flush=True)
    probe_check(lib, lib.ts_probe_lds(src.data_ptr(), perm.data_ptr(), dma.data_ptr(), tr.data_ptr(),
                                buf.data_ptr(), valid, _lib.stream_of(src)), "ts_probe_lds")
    torch.cuda.synchronize()
    got = dma.view(64, 4).cpu().numpy()
    p = perm.cpu().numpy()
    # lane i's 16 bytes land at LDS offset 16 i
    np.testing.assert_array_equal(got, np.stack([np.arange(4 * j, 4 * j + 4) for j in p]))
    # buffer DMA: lane i's 16 bytes at LDS offset 16 i; a lane wholly past the
    # resource's range writes zeros (the kernels rely on this for ragged tiles)
    gotb = buf.view(64, 4).cpu().numpy()
    print("buffer DMA straddling lane:", gotb[int(np.where(p == 37)[0][0])].tolist(), flush=True)
    for lane, j in enumerate(p):
        if 16 * j + 16 <= valid:
            np.testing.assert_array_equal(gotb[lane], np.arange(4 * j, 4 * j + 4), err_msg=f"lane {lane}")
        elif 16 * j >= valid:
            np.testing.assert_array_equal(gotb[lane], np.zeros(4), err_msg=f"lane {lane}")
    t = tr.view(64, 4).cpu().numpy().astype(np.int64)
    print("ds_read_b64_tr_b16 lanes 0..19:", t[:20].tolist(), flush=True)
    # within each group of 16 lanes the four values come from four different
    # 8-byte rows of that group (a transpose), never from another group
    for lane in range(64):
        rows = set((t[lane] // 4).tolist())
        assert all(16 * (lane // 16) <= r < 16 * (lane // 16) + 16 for r in rows), (lane, t[lane])


def test_cross_row_lane_reductions(cuda):
    """rows_max4 / rows_sum4 combine lanes l, l^16, l^32, l^48 (the attention
    softmax's column reductions), pinned against numpy on distinct values."""
    lib = probe_library()
    x = np.random.default_rng(5).permutation(64).astype(np.float32) - 20.0
    src = torch.tensor(x, device=cuda)
    out = torch.empty(6 * 64, dtype=torch.float32, device=cuda)
    print("probe: ts_probe_lanes", flush=True)
    probe_check(lib, lib.ts_probe_lanes(src.data_ptr(), out.data_ptr(), _lib.stream_of(src)), "ts_probe_lanes")
    torch.cuda.synchronize()
    got = out.view(6, 64).cpu().numpy()
    rows = x.reshape(4, 16)
    np.testing.assert_array_equal(got[0], np.tile(rows.max(axis=0), 4))
    np.testing.assert_array_equal(got[1], np.tile(rows.sum(axis=0), 4))
    # each swap pairs rows 0/1 and 2/3 (16) or the two halves (32); together
    # the two results of one swap hold both members of every pair
    for k, partner in ((2, 16), (4, 32)):
        pair = np.sort(np.stack([got[k], got[k + 1]]), axis=0)
        want = np.sort(np.stack([x, x[np.arange(64) ^ partner]]), axis=0)
        np.testing.assert_array_equal(pair, want)
    print("permlane16_swap:", got[2][:20].tolist(), got[3][:20].tolist(), flush=True)


def test_buffer_dma_instruction_offset_moves_both_addresses(cuda):
    """buffer_load_dwordx4 ... lds with an immediate instruction offset: the
    offset is added to the LDS destination as well as to the global address,
    so one M0 value serves DMA instructions whose LDS and global offsets
    advance together (lane i's 16 bytes from byte 1024 + 16 i land at LDS
    byte 1024 + 16 i; the first 1 KB of the block is left alone)."""
    lib = probe_library()
    src = torch.arange(128 * 4, dtype=torch.int32, device=cuda)
    out = torch.empty(128 * 4, dtype=torch.int32, device=cuda)
    print("probe: ts_probe_dma_offset", flush=True)
    probe_check(lib, lib.ts_probe_dma_offset(src.data_ptr(), out.data_ptr(), _lib.stream_of(src)),
                "ts_probe_dma_offset")
    torch.cuda.synchronize()
    got = out.view(128, 4).cpu().numpy()
    print("dma offset: LDS rows 0, 64:", got[0].tolist(), got[64].tolist(), flush=True)
    untouched = np.full((64, 4), np.int32(np.uint32(0xDEADBEEF).view(np.int32)))
    np.testing.assert_array_equal(got[:64], untouched)
    np.testing.assert_array_equal(got[64:], np.arange(256, 512).reshape(64, 4))
