"""Record stock-module RMSNorm bytes on the GPU as a data-only fixture.

Run on a GPU box (it needs torch's GPU kernels, whose summation order and
rsqrt rounding are what the fixture records):

    python tests/golden/make_rmsnorm_golden.py gpurun_out/rmsnorm_device.npz

For each case it draws ``hidden`` [rows, width] from a seeded CPU generator,
runs transformers' stock ``Qwen3RMSNorm`` (the module the reference's swap
must reproduce byte for byte, reference tests/test_rms_norm_precision.py:27-39)
and ``torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + eps)`` (the
statistic the reference's FP32RMSNormVJP saves, accel/rms_norm.py:11-13) on
cuda:0, and keeps up to eight rows of each as raw dtype bits (the row
indices are stored: a row's result depends on its own values, the tensor's
row count and width, and its position).  Nothing from the reference is imported.
"""

from __future__ import annotations

import sys

import numpy as np
import torch

CASES = [  # (rows, width, dtype, eps)
    (64, 128, "bfloat16", 1e-6), (64, 128, "float16", 1e-6), (64, 128, "float32", 1e-6),
    (1, 128, "bfloat16", 1e-6), (3, 128, "bfloat16", 1e-6), (16, 128, "bfloat16", 1e-5),
    (16384 * 8, 128, "bfloat16", 1e-6), (16384, 4096, "bfloat16", 1e-6),
    (1, 4096, "bfloat16", 1e-6), (2, 4096, "bfloat16", 1e-6), (3, 4096, "float16", 1e-6),
    (5, 4096, "bfloat16", 1e-6), (8, 4096, "float32", 1e-6), (7, 64, "bfloat16", 1e-6),
    (64, 64, "bfloat16", 1e-6), (64, 32, "float16", 1e-6), (64, 16, "bfloat16", 1e-6),
    (64, 8192, "bfloat16", 1e-6), (3, 8192, "bfloat16", 1e-6), (16, 5120, "bfloat16", 1e-6),
    (64, 256, "bfloat16", 1e-6), (64, 1024, "bfloat16", 1e-6), (2, 2048, "bfloat16", 1e-6),
    (4, 100, "bfloat16", 1e-6), (64, 96, "bfloat16", 1e-6), (64, 130, "bfloat16", 1e-6),
    (64, 132, "bfloat16", 1e-6), (64, 1000, "float16", 1e-6), (16, 16384, "bfloat16", 1e-6),
    (8, 11008, "bfloat16", 1e-6), (1, 1024, "bfloat16", 1e-6), (5, 3, "bfloat16", 1e-6),
    (33, 2, "float32", 1e-6),
]


def main(path: str) -> None:
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    dev = torch.device("cuda:0")
    out: dict[str, np.ndarray] = {}
    meta = []
    for i, (rows, width, dt, eps) in enumerate(CASES):
        dtype = getattr(torch, dt)
        g = torch.Generator().manual_seed(1000 + i)
        hidden = torch.randn(rows, width, generator=g).to(dtype)
        # a few rows far from unit scale, so the variance spans binades
        hidden[: min(rows, 2)] *= 37.0
        weight = torch.linspace(0.4, 3.0, width).to(dtype)
        module = Qwen3RMSNorm(width, eps=eps).to(dev, dtype)
        with torch.no_grad():
            module.weight.copy_(weight.to(dev))
            h = hidden.to(dev)
            primal = module(h)
            rstd = torch.rsqrt(h.float().pow(2).mean(-1, keepdim=True) + eps)
        torch.cuda.synchronize()
        keep = np.unique(np.linspace(0, rows - 1, min(rows, 8)).round().astype(np.int64))
        bits = torch.int16 if dtype != torch.float32 else torch.int32
        out[f"hidden_{i}"] = hidden[keep].view(bits).numpy()
        out[f"primal_{i}"] = primal[keep].cpu().view(bits).numpy()
        out[f"rstd_{i}"] = rstd[keep, 0].cpu().numpy()
        out[f"rows_index_{i}"] = keep
        meta.append((rows, width, ["float32", "float16", "bfloat16"].index(dt), eps))
        print(f"case {i}: rows={rows} width={width} {dt}", flush=True)
    out["meta"] = np.array(meta, dtype=np.float64)
    np.savez_compressed(path, **out)
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "rmsnorm_device.npz")
