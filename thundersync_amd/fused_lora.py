"""LoRA linear layers evaluated against a merged effective weight, on gfx950.

Interface of the reference's ``accel/fused_lora.py`` (``FusedLoRALinear``,
``fuse_merged_lora_forward``, ``unfuse_merged_lora_forward``): with the
frozen base weight ``W`` and the adapters ``A`` ([rank, in]) and ``B``
([out, rank]) merged in place (``W_eff = W + s B A``), the forward is one
GEMM and the backward the exact derivative of the unmerged layer:

    y = x W_eff^T      dx = g W_eff      dA = s (g B)^T x      dB = s g^T (x A^T)

Every product runs in the library (``ts_lora_fwd`` / ``ts_lora_bwd``, bf16 or
fp16 operands on MFMA with fp32 accumulation); the adapter gradients come back as
fp32 sums over fixed row ranges added in order, so a call gives the same
bytes every time, and are cast to each adapter's own dtype.  The adapters
are cast to the activation dtype before the products, as the reference does.

Activations must be bf16 or fp16 CUDA tensors (the weight of the same dtype)
with ``in`` and ``out`` multiples of 8;
anything else raises -- there is no host fallback.  ``fuse_merged_lora_forward``
converts only the layers that meet this (and leaves the rest as they were).  The caller merges before
and unmerges after (the optimizer step moves A and B and leaves the merged
weight stale), which the two module-level functions do through the layer's
own ``merge`` / ``unmerge`` (PEFT's ``LoraLayer`` API).
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .operator_profiling import device_role, operator_range

__all__ = ["FusedLoRALinear", "fuse_merged_lora_forward", "unfuse_merged_lora_forward"]

# attribute names on a converted layer (the flag keeps the reference's name)
_FLAG = "_thundersync_fused"
_SAVED_FORWARD = "_thundersync_unfused_forward"


def _rows_view(t: torch.Tensor, features: int, name: str) -> torch.Tensor:
    """``t`` as [rows, features] with a unit inner stride, without a copy when possible."""
    if t.shape[-1] != features:
        raise ValueError(f"{name} has {t.shape[-1]} features, expected {features}")
    rows = t.reshape(-1, features)
    if rows.stride(1) != 1 or rows.stride(0) % 8 or rows.data_ptr() % 16 or rows.stride(0) < features:
        rows = rows.contiguous()
    return rows


def _check(x: torch.Tensor, weight: torch.Tensor) -> None:
    if not x.is_cuda:
        raise RuntimeError("thundersync_amd FusedLoRALinear runs on the GPU only; got a CPU tensor")
    if x.dtype not in (torch.bfloat16, torch.float16) or weight.dtype != x.dtype:
        raise TypeError(f"FusedLoRALinear takes bf16 or fp16 activations and a weight of the same dtype, got "
                        f"{x.dtype} / {weight.dtype}")
    if weight.dim() != 2:
        raise ValueError(f"weight must be [out, in], got {tuple(weight.shape)}")
    out_f, in_f = weight.shape
    if in_f % 8 or out_f % 8:
        raise ValueError(f"in ({in_f}) and out ({out_f}) features must be multiples of 8")
    if weight.device != x.device:
        raise ValueError("x and weight must be on the same device")


def _weight_rows(weight: torch.Tensor) -> torch.Tensor:
    if weight.stride(1) != 1 or weight.stride(0) % 8 or weight.data_ptr() % 16:
        return weight.contiguous()
    return weight


class FusedLoRALinear(torch.autograd.Function):
    """``x @ W_eff.T`` with adapter gradients, no adapter GEMM in forward
    (accel/fused_lora.py:26-48)."""

    @staticmethod
    def forward(ctx, x, weight, lora_a, lora_b, scaling):
        _check(x, weight)
        out_f, in_f = weight.shape
        rows = _rows_view(x, in_f, "x")
        w = _weight_rows(weight)
        y = torch.empty(rows.shape[0], out_f, dtype=x.dtype, device=x.device)
        lib = _lib.require_library()
        with operator_range("fused_lora_forward", role=device_role(x.device), rows=rows.shape[0], inp=in_f,
                            out=out_f):
            _lib.check(
                lib.ts_lora_fwd(rows.data_ptr(), rows.stride(0), w.data_ptr(), w.stride(0), rows.shape[0], in_f,
                                out_f, y.data_ptr(), y.stride(0), _lib.dtype_code(x.dtype), _lib.stream_of(x)),
                f"ts_lora_fwd(rows={rows.shape[0]}, in={in_f}, out={out_f})",
            )
        ctx.save_for_backward(x, weight, lora_a, lora_b)
        ctx.scaling = float(scaling)
        return y.view(*x.shape[:-1], out_f)

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_out):
        x, weight, lora_a, lora_b = ctx.saved_tensors
        out_f, in_f = weight.shape
        rank = lora_a.shape[0]
        if lora_a.shape != (rank, in_f) or lora_b.shape != (out_f, rank):
            raise ValueError(f"adapters {tuple(lora_a.shape)} / {tuple(lora_b.shape)} do not fit weight "
                             f"{tuple(weight.shape)}")
        want_x, want_a, want_b = ctx.needs_input_grad[0], ctx.needs_input_grad[2], ctx.needs_input_grad[3]
        rows = _rows_view(x, in_f, "x")
        g = _rows_view(grad_out.to(x.dtype), out_f, "grad_out")
        n = rows.shape[0]
        dev = x.device
        # the products run in the activation dtype (accel/fused_lora.py:40-43);
        # B is handed over transposed, [rank, out]
        a = lora_a.detach().to(x.dtype).contiguous() if want_b else None
        b_t = lora_b.detach().to(x.dtype).t().contiguous() if want_a else None
        w = _weight_rows(weight) if want_x else None
        dx = torch.empty(n, in_f, dtype=x.dtype, device=dev) if want_x else None
        da = torch.empty(rank, in_f, dtype=torch.float32, device=dev) if want_a else None
        db = torch.empty(out_f, rank, dtype=torch.float32, device=dev) if want_b else None
        lib = _lib.require_library()
        ws_bytes = lib.ts_lora_bwd_workspace(n, in_f, out_f, rank)
        ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=dev)
        with operator_range("fused_lora_backward", role=device_role(dev), rows=n, inp=in_f, out=out_f, rank=rank):
            _lib.check(
                lib.ts_lora_bwd(g.data_ptr(), g.stride(0), rows.data_ptr(), rows.stride(0), _lib.ptr(w),
                                w.stride(0) if w is not None else 0, _lib.ptr(a), _lib.ptr(b_t), rank,
                                ctypes.c_float(ctx.scaling), n, in_f, out_f, _lib.ptr(dx),
                                dx.stride(0) if dx is not None else 0, _lib.ptr(da), _lib.ptr(db), ws.data_ptr(),
                                ws_bytes, _lib.dtype_code(x.dtype), _lib.stream_of(x)),
                f"ts_lora_bwd(rows={n}, in={in_f}, out={out_f}, rank={rank})",
            )
        grad_x = dx.view(x.shape) if dx is not None else None
        grad_a = da.to(lora_a.dtype) if da is not None else None
        grad_b = db.to(lora_b.dtype) if db is not None else None
        return grad_x, None, grad_a, grad_b, None


def _active_adapter(model: torch.nn.Module, *, strict: bool) -> str:
    adapter = getattr(model, "active_adapter", "default")
    if isinstance(adapter, (list, tuple)):
        if strict and len(adapter) != 1:
            raise ValueError("fused LoRA supports one active adapter")
        adapter = adapter[0]
    return adapter


def _adapter_of(layer: torch.nn.Module, adapter: str):
    """(A weight, B weight, scaling) of ``adapter`` on a LoRA layer, or None when
    the layer has no such adapter or would drop out inputs (a merged weight
    cannot reproduce dropout; accel/fused_lora.py:51-67)."""
    a_dict, b_dict = getattr(layer, "lora_A", None), getattr(layer, "lora_B", None)
    if a_dict is None or b_dict is None or adapter not in a_dict or adapter not in b_dict:
        return None
    drops = getattr(layer, "lora_dropout", None)
    if drops is not None and adapter in drops and getattr(drops[adapter], "p", 0.0):
        return None
    scale = float(getattr(layer, "scaling", {}).get(adapter, 1.0))
    return a_dict[adapter].weight, b_dict[adapter].weight, scale


# largest adapter rank the backward's rank products take (ts_lora_bwd)
MAX_RANK = 256


def fusable(base: torch.nn.Linear, a_weight: torch.Tensor, b_weight: torch.Tensor) -> bool:
    """Whether the kernels can run a layer: a bf16 or fp16 GPU base weight
    with ``in`` and ``out`` multiples of 8, adapters on its device that fit
    it, a rank of at most :data:`MAX_RANK`, and a loaded library.  A layer
    that fails stays unmerged and keeps its own forward."""
    w = base.weight
    if not w.is_cuda or w.dtype not in (torch.bfloat16, torch.float16) or w.dim() != 2:
        return False
    out_f, in_f = w.shape
    rank = a_weight.shape[0] if a_weight.dim() == 2 else -1
    if in_f % 8 or out_f % 8 or not 0 < rank <= MAX_RANK:
        return False
    if tuple(a_weight.shape) != (rank, in_f) or tuple(b_weight.shape) != (out_f, rank):
        return False
    if a_weight.device != w.device or b_weight.device != w.device:
        return False
    return _lib.library() is not None


def fuse_merged_lora_forward(peft_model: torch.nn.Module) -> int:
    """Merge each LoRA layer's active adapter into its base weight in place and
    route the layer through :class:`FusedLoRALinear`; returns how many layers
    were converted (accel/fused_lora.py:70-108).  Layers the kernels cannot
    run (:func:`fusable`) are left unmerged and unconverted.  Call
    :func:`unfuse_merged_lora_forward` before the optimizer step."""
    adapter = _active_adapter(peft_model, strict=True)
    converted = 0
    for layer in peft_model.modules():
        if getattr(layer, _FLAG, False):
            continue
        base = getattr(layer, "base_layer", None)
        parts = _adapter_of(layer, adapter)
        if parts is None or not isinstance(base, torch.nn.Linear):
            continue
        if not fusable(base, parts[0], parts[1]):
            continue
        layer.merge(adapter_names=[adapter])
        a_weight, b_weight, scale = parts

        def fused(x, _base=base, _a=a_weight, _b=b_weight, _s=scale):
            return FusedLoRALinear.apply(x, _base.weight, _a, _b, _s)

        setattr(layer, _SAVED_FORWARD, layer.forward)
        layer.forward = fused
        setattr(layer, _FLAG, True)
        converted += 1
    return converted


def unfuse_merged_lora_forward(peft_model: torch.nn.Module) -> int:
    """Restore each converted layer's own forward and unmerge its adapter, so the
    optimizer step sees plain base weights (accel/fused_lora.py:111-126)."""
    restored = 0
    for layer in peft_model.modules():
        if not getattr(layer, _FLAG, False):
            continue
        layer.forward = getattr(layer, _SAVED_FORWARD)
        delattr(layer, _SAVED_FORWARD)
        setattr(layer, _FLAG, False)
        layer.unmerge()
        restored += 1
    return restored
