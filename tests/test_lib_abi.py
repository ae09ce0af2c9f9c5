"""The C-ABI library builds, loads, and exports what include/*.h declares.

CPU-only: loading libthundersync_hip.so and calling the version/error
entry points touches no GPU.
"""

from __future__ import annotations

import ctypes
import re

from tests.conftest import ROOT
from thundersync_amd import _lib


def declared_symbols() -> set[str]:
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names.update(re.findall(r"\b(ts_[a-z0-9_]+)\s*\(", text))
    return names


def test_every_declared_symbol_has_a_binding():
    assert declared_symbols() == set(_lib.SIGNATURES)


def test_the_library_loads_and_exports_every_symbol():
    assert _lib.LIB_PATH.exists(), "build the library first (__graft_entry__.build())"
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_version_and_empty_error(monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "auto")
    _lib.reset()
    try:
        lib = _lib.require_library()
        assert lib.ts_hip_version().decode().startswith("thundersync_hip")
        assert "gfx950" in _lib.hip_build()
    finally:
        _lib.reset()


def test_argument_errors_are_reported_without_a_device(monkeypatch):
    """A null pointer is refused before any launch; the message names the call."""
    monkeypatch.setenv(_lib.HIP_ENV, "auto")
    _lib.reset()
    try:
        lib = _lib.require_library()
        status = lib.ts_rmsnorm_fwd(None, None, None, None, 4, 8, 1e-6, _lib.TS_BF16, None)
        assert status != 0
        assert "ts_rmsnorm_fwd" in lib.ts_hip_last_error().decode()
        try:
            _lib.check(status, "ts_rmsnorm_fwd(test)")
        except RuntimeError as error:
            assert "null pointer" in str(error)
        else:  # pragma: no cover
            raise AssertionError("check() did not raise")
    finally:
        _lib.reset()


def test_the_operator_library_exports_no_test_probes():
    """The hardware probes live in the test-only tests/probe/libts_probe.so."""
    from tests.probe.build_probe import LIB_PATH as PROBE_LIB

    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in ("ts_probe_layouts", "ts_probe_lds", "ts_probe_lanes"):
        assert not hasattr(lib, name), name
    assert PROBE_LIB.exists(), "build the probe library first (__graft_entry__.build())"
    probe = ctypes.CDLL(str(PROBE_LIB))
    for name in ("ts_probe_layouts", "ts_probe_lds", "ts_probe_lanes", "ts_probe_last_error"):
        assert hasattr(probe, name), name


def test_work_item_sizes_match_the_host_mirrors(monkeypatch):
    """ts_attn_q_block / ts_attn_kv_block agree with the layout's mirrors for
    every GQA group and head dim the kernels take (the library validates
    each problem's q_block / kv_block against them)."""
    from thundersync_amd import attention as att

    monkeypatch.setenv(_lib.HIP_ENV, "auto")
    _lib.reset()
    try:
        lib = _lib.require_library()
        for group in (1, 2, 3, 4, 5, 6, 8):
            assert lib.ts_attn_q_block(group) == att.q_block_rows(group, 1)
            for head_dim in att.HEAD_DIMS:
                assert lib.ts_attn_kv_block(group, head_dim) == att.kv_block_keys(group, 1, head_dim), (group, head_dim)
    finally:
        _lib.reset()
