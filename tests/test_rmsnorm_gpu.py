"""RMSNorm HIP kernels against the CPU oracle (accel/rms_norm.py restated).

Bars: the primal within two units in the last place of the output dtype
(the fp32 sum of squares is reduced in a different order than torch's, which
can move rstd by an ulp; the primal rounds twice -- xhat to the dtype, then
w * xhat -- and each rounding can then land one unit apart); rstd within 2e-6
relative; dx and dw (fp32 VJP, cast once) within the output dtype's rounding
of the fp64 closed form.  dW is a fixed-order reduction: two runs are
bit-identical.
"""

from __future__ import annotations

import pytest
import torch

from oracle import rms_norm as ref
from thundersync_amd.rms_norm import FP32RMSNormVJP, rms_norm_backward, rms_norm_forward

pytestmark = pytest.mark.gpu

SHAPES = [(3, 128), (129, 128), (64, 4096), (257, 4096), (16, 32), (7, 40), (5, 200), (2, 5), (33, 8192), (4, 12288),
          # backward variants: 8 vectors per lane, part empty (3584); 16 vectors, part empty, four
          # waves (5120); 282 partial rows of 32 (9000 x 1024); 1024 partial rows of 69 rows (70000 x 128)
          (37, 3584), (19, 5120), (9000, 1024), (70000, 128)]


def ulp(dtype):
    return {torch.bfloat16: 2 ** -7, torch.float16: 2 ** -10, torch.float32: 2 ** -23}[dtype]


def make(rows, width, dtype, device, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, width, generator=g).to(dtype)
    w = torch.linspace(0.4, 3.0, width).to(dtype)
    dy = torch.randn(rows, width, generator=g).to(dtype)
    return x, w, dy


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,width", SHAPES)
def test_forward_matches_oracle(cuda, rows, width, dtype):
    print(f"rmsnorm fwd rows={rows} width={width} {dtype}", flush=True)
    x, w, _ = make(rows, width, dtype, cuda, rows * 31 + width)
    want, want_rstd = ref.rms_norm_forward(x, w, 1e-6)
    got, rstd = rms_norm_forward(x.to(cuda), w.to(cuda), 1e-6)
    torch.cuda.synchronize()
    torch.testing.assert_close(rstd.cpu(), want_rstd, rtol=2e-6, atol=0)
    # two output units for 16-bit outputs; fp32 outputs carry rstd's own
    # reduction-order difference (a few fp32 ulps)
    units = 2.02 if dtype != torch.float32 else 8.0
    tol = want.float().abs() * ulp(dtype) * units + 1e-30
    err = (got.cpu().float() - want.float()).abs()
    assert bool((err <= tol).all()), float((err / tol).max())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,width", SHAPES)
def test_backward_matches_closed_form(cuda, rows, width, dtype):
    print(f"rmsnorm bwd rows={rows} width={width} {dtype}", flush=True)
    x, w, dy = make(rows, width, dtype, cuda, rows * 17 + width)
    _, rstd = ref.rms_norm_forward(x, w, 1e-6)
    want_dx, want_dw = ref.rms_norm_backward_closed_form(dy, x, w, rstd)
    dx, dw = rms_norm_backward(dy.to(cuda), x.to(cuda), w.to(cuda), rstd.to(cuda))
    dx2, dw2 = rms_norm_backward(dy.to(cuda), x.to(cuda), w.to(cuda), rstd.to(cuda))
    torch.cuda.synchronize()
    assert torch.equal(dw, dw2) and torch.equal(dx, dx2)
    # fp32 arithmetic then one rounding to the dtype
    scale_dx = want_dx.abs().max().item()
    torch.testing.assert_close(dx.cpu().double(), want_dx, rtol=2 * ulp(dtype), atol=1e-5 * scale_dx + 1e-12)
    scale_dw = want_dw.abs().max().item()
    torch.testing.assert_close(dw.cpu().double(), want_dw, rtol=2 * ulp(dtype), atol=max(1e-5, ulp(dtype)) * scale_dw)


def test_autograd_function_and_partial_needs(cuda):
    x, w, dy = make(65, 4096, torch.bfloat16, cuda, 5)
    xc = x.to(cuda).requires_grad_()
    wc = w.to(cuda).requires_grad_()
    y = FP32RMSNormVJP.apply(xc, wc, 1e-6)
    y.backward(dy.to(cuda))
    want_y, rstd = ref.rms_norm_forward(x, w, 1e-6)
    want_dx, want_dw = ref.rms_norm_backward(dy, x, w, 1e-6)
    assert (y.detach().cpu().float() - want_y.float()).abs().max().item() <= 2 ** -7 * 3 * 4
    torch.testing.assert_close(xc.grad.cpu().float(), want_dx.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(wc.grad.cpu().float(), want_dw.float(), rtol=2e-2, atol=1e-1)
    # dx only
    dx, dw = rms_norm_backward(dy.to(cuda), x.to(cuda), w.to(cuda), rstd.to(cuda), (True, False))
    assert dw is None and dx is not None
    dx, dw = rms_norm_backward(dy.to(cuda), x.to(cuda), w.to(cuda), rstd.to(cuda), (False, True))
    assert dx is None and dw is not None


def test_cpu_tensors_are_refused():
    x = torch.randn(2, 8, dtype=torch.bfloat16)
    w = torch.ones(8, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        rms_norm_forward(x, w, 1e-6)
