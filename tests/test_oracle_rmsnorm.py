"""Pin the RMSNorm oracle (CPU).

``oracle.rms_norm.device_forward`` restates the stock forward as the GPU
computes it (torch's reduction schedule for the variance, correctly rounded
rsqrt).  It is checked bit for bit against stock ``Qwen3RMSNorm`` outputs and
saved statistics recorded on an MI355X (tests/golden/rmsnorm_device.npz,
written by tests/golden/make_rmsnorm_golden.py), and against an fp64 sum
within fp32 rounding.  A dropped term, a different pairing or a /width in
place of MeanOps' *factor changes bits on these rows.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import rms_norm as ref

GOLDEN = Path(__file__).resolve().parent / "golden" / "rmsnorm_device.npz"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _cases():
    data = np.load(GOLDEN)
    for i, (rows, width, code, eps) in enumerate(data["meta"]):
        yield i, int(rows), int(width), DTYPES[int(code)], float(eps), data


def _tensor(bits: np.ndarray, dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits)).view(dtype)


@pytest.mark.parametrize("case", list(range(33)))
def test_device_forward_matches_recorded_gpu_bytes(case):
    for i, rows, width, dtype, eps, data in _cases():
        if i != case:
            continue
        hidden = _tensor(data[f"hidden_{i}"], dtype)
        want = _tensor(data[f"primal_{i}"], dtype)
        want_rstd = data[f"rstd_{i}"]
        index = data[f"rows_index_{i}"]
        weight = torch.linspace(0.4, 3.0, width).to(dtype)
        sums = ref.device_row_sums(hidden.float().numpy(), rows=rows, row_index=index)
        rstd = ref.device_rstd(sums, rows, width, eps)
        assert np.array_equal(rstd.view(np.int32), want_rstd.view(np.int32)), (rows, width, dtype)
        xhat = (hidden.float() * torch.from_numpy(rstd)[:, None]).to(dtype)
        assert torch.equal(weight * xhat, want), (rows, width, dtype)
        # fp32 rounding of the exact sum: each of the width additions rounds once
        exact = (hidden.double() ** 2).sum(-1).numpy()
        assert np.all(np.abs(sums - exact) <= exact * width * 2.0 ** -23 + 1e-30)
        return
    pytest.skip("no such case")


def test_device_forward_whole_tensor_path():
    """device_forward on a whole tensor equals the per-row restatement."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(9, 130, generator=g).to(torch.bfloat16)
    w = torch.linspace(0.4, 3.0, 130).to(torch.bfloat16)
    y, rstd = ref.device_forward(x, w, 1e-6)
    sums = ref.device_row_sums(x.float().numpy())
    assert np.array_equal(rstd[:, 0].numpy(), ref.device_rstd(sums, 9, 130, 1e-6))
    # and within two bf16 roundings of the fp64 formula
    closed = w.double() * x.double() * torch.rsqrt(x.double().pow(2).mean(-1, keepdim=True) + 1e-6)
    assert bool(((y.double() - closed).abs() <= closed.abs() * 2.0 ** -7 * 2.02).all())


def test_schedule_matches_known_configurations():
    # (rows, width) -> (vec, bw, bh, ym, step) as Reduce.cuh derives them on 256 CUs
    assert ref.device_reduce_schedule(64, 128) == (True, 32, 1, 0, 32)
    assert ref.device_reduce_schedule(16384, 4096) == (True, 64, 1, 0, 64)
    assert ref.device_reduce_schedule(1, 4096) == (True, 512, 1, 0, 512)
    assert ref.device_reduce_schedule(4, 4096) == (True, 128, 1, 0, 128)
    assert ref.device_reduce_schedule(64, 8192) == (True, 64, 8, 64, 512)
    assert ref.device_reduce_schedule(64, 100) == (False, 64, 1, 0, 64)
    assert ref.device_reduce_schedule(1, 1 << 18) is None
