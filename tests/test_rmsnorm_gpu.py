"""RMSNorm HIP kernels against the CPU oracle (accel/rms_norm.py restated).

Bars: the primal and rstd bit-identical (rtol = atol = 0) to the oracle's
restatement of the GPU forward and to torch's own stock operations on the
same device -- the reference's "original primal bytes" contract
(tests/test_rms_norm_precision.py:27-39); dx and dw (fp32 VJP, cast once)
within the output dtype's rounding of the fp64 closed form.  dW is a
fixed-order reduction: two runs are bit-identical.
"""

from __future__ import annotations

import pytest
import torch

from oracle import rms_norm as ref
from thundersync_amd.rms_norm import FP32RMSNormVJP, rms_norm_backward, rms_norm_forward

pytestmark = pytest.mark.gpu

SHAPES = [(3, 128), (129, 128), (64, 4096), (257, 4096), (16, 32), (7, 40), (5, 200), (2, 5), (33, 8192), (4, 12288),
          # forward schedules: one row over 512 threads; 256; 128 threads and a split row; misaligned
          # rows (width % 4 != 0, >= 128); scalar loads over 64 lanes with a second element
          (1, 4096), (2, 2048), (4, 12288), (9, 130), (64, 100),
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
    x[: min(rows, 3)] *= 23.0  # rows far from unit scale
    want, want_rstd = ref.device_forward(x, w, 1e-6)
    got, rstd = rms_norm_forward(x.to(cuda), w.to(cuda), 1e-6)
    # torch's own operations on the device (the stock module's forward)
    xs = x.to(cuda).to(torch.float32)
    stock_rstd = torch.rsqrt(xs.pow(2).mean(-1, keepdim=True) + 1e-6)
    stock = w.to(cuda) * (xs * stock_rstd).to(dtype)
    torch.cuda.synchronize()
    assert torch.equal(rstd, stock_rstd) and torch.equal(got, stock)
    assert torch.equal(rstd.cpu(), want_rstd) and torch.equal(got.cpu(), want)
    # and within two output roundings of the fp64 formula
    closed = w.double() * (x.double() * torch.rsqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-6))
    # (plus the absolute spacing of fp16 subnormals, which tiny outputs round to)
    tol = closed.abs() * ulp(dtype) * 2.02 + torch.finfo(dtype).tiny * ulp(dtype) * 8
    assert bool(((got.cpu().double() - closed).abs() <= tol).all())


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
