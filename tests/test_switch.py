"""THUNDERSYNC_HIP = require | off | auto, with THUNDERSYNC_FA4's semantics.

Mirrors the reference's switch tests (tests/test_fa4_switch.py:36-62): `off`
never loads, `require` raises at every resolution while the library cannot
load, `auto` leaves the path absent, unknown settings are refused.
"""

from __future__ import annotations

import pytest

from thundersync_amd import _lib


@pytest.fixture
def unresolved(monkeypatch):
    _lib.reset()
    yield
    _lib.reset()


def test_off_never_loads(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "off")
    called = []
    monkeypatch.setattr(_lib, "_load", lambda: called.append(1))
    assert _lib.library() is None
    assert _lib.hip_build() is None
    assert called == []
    with pytest.raises(RuntimeError, match="switched off"):
        _lib.require_library()


def test_require_without_a_library_raises_every_time(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "require")

    def missing():
        raise OSError("not built")

    monkeypatch.setattr(_lib, "_load", missing)
    for _ in range(2):
        with pytest.raises(RuntimeError, match="THUNDERSYNC_HIP=require"):
            _lib.library()
    assert _lib._RESOLVED is False
    assert _lib.hip_build() is None


def test_auto_without_a_library_leaves_it_absent(unresolved, monkeypatch):
    monkeypatch.delenv(_lib.HIP_ENV, raising=False)

    def missing():
        raise OSError("not built")

    monkeypatch.setattr(_lib, "_load", missing)
    assert _lib.hip_setting() == "auto"
    assert _lib.library() is None
    assert _lib._RESOLVED is True
    with pytest.raises(RuntimeError, match="not available"):
        _lib.require_library()


def test_an_unknown_setting_is_refused(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "maybe")
    with pytest.raises(ValueError, match="THUNDERSYNC_HIP"):
        _lib.library()


def test_require_with_the_library_resolves_once(unresolved, monkeypatch):
    monkeypatch.setenv(_lib.HIP_ENV, "require")
    lib = _lib.library()
    assert lib is not None and _lib.library() is lib
    assert _lib.hip_build().startswith("thundersync_hip")
