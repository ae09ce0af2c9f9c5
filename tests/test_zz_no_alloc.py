"""ts_rmsnorm_bwd_noalloc: the RMSNorm backward with its dW partials in a
file-scope device array, against ts_rmsnorm_bwd with a caller workspace.

Bar: bit-identical dx and dw (same kernels, same fixed-order dW reduction),
on two calls in a row -- the second smaller, so stale partials of the first
would show -- for each dtype; sizes beyond the array are refused before any
launch.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from thundersync_amd import _lib
from thundersync_amd.rms_norm import rms_norm_backward, rms_norm_forward

pytestmark = pytest.mark.gpu


def _noalloc(lib, dy, x, w, rstd, dx, dw):
    rows, width = x.shape
    status = lib.ts_rmsnorm_bwd_noalloc(
        dy.data_ptr(), x.data_ptr(), w.data_ptr(), rstd.data_ptr(), _lib.ptr(dx), _lib.ptr(dw),
        rows, width, _lib.dtype_code(x.dtype), _lib.stream_of(x),
    )
    _lib.check(status, f"ts_rmsnorm_bwd_noalloc(rows={rows}, width={width})")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_noalloc_matches_workspace_entry_point(cuda, dtype):
    lib = _lib.require_library()
    for rows, width in [(8192, 4096), (300, 4096), (70000, 128), (5, 130)]:
        print(f"noalloc rmsnorm bwd rows={rows} width={width} {dtype}", flush=True)
        g = torch.Generator().manual_seed(rows + width)
        x = torch.randn(rows, width, generator=g).to(dtype).to(cuda)
        dy = torch.randn(rows, width, generator=g).to(dtype).to(cuda)
        w = torch.linspace(0.4, 3.0, width).to(dtype).to(cuda)
        _, rstd = rms_norm_forward(x, w, 1e-6)
        want_dx, want_dw = rms_norm_backward(dy, x, w, rstd)
        dx = torch.empty_like(x)
        dw = torch.empty_like(w)
        _noalloc(lib, dy, x, w, rstd, dx, dw)
        torch.cuda.synchronize()
        assert torch.equal(dx, want_dx) and torch.equal(dw, want_dw)
        # dx alone and dw alone
        dx2 = torch.empty_like(x)
        _noalloc(lib, dy, x, w, rstd, dx2, None)
        dw2 = torch.empty_like(w)
        _noalloc(lib, dy, x, w, rstd, None, dw2)
        torch.cuda.synchronize()
        assert torch.equal(dx2, want_dx) and torch.equal(dw2, want_dw)


def test_noalloc_refuses_sizes_beyond_the_array(cuda):
    lib = _lib.require_library()
    x = torch.empty(1, 8, dtype=torch.bfloat16, device=cuda)
    rows, width = 1 << 20, 16384  # 256 partial rows of 16384 fp32 = 16 MiB
    need = lib.ts_rmsnorm_bwd_workspace(rows, width)
    assert need > 8 << 20
    status = lib.ts_rmsnorm_bwd_noalloc(x.data_ptr(), x.data_ptr(), x.data_ptr(), x.data_ptr(), None,
                                        x.data_ptr(), rows, width, _lib.TS_BF16, _lib.stream_of(x))
    assert status == 1
    assert "scratch array" in lib.ts_hip_last_error().decode()
