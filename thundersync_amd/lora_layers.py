"""A LoRA linear layer with the slice of PEFT's ``LoraLayer`` API that the
merged-weight path drives, for models built without PEFT.

:func:`~thundersync_amd.fused_lora.fuse_merged_lora_forward` reads a layer's
``base_layer`` (an ``nn.Linear``), the ``lora_A`` / ``lora_B`` /
``lora_dropout`` module dicts and the ``scaling`` dict, and calls
``merge(adapter_names=[...])`` / ``unmerge()``; :class:`LoraLinear` provides
exactly that, with PEFT's conventions: ``A`` is ``[rank, in]``, ``B`` is
``[out, rank]`` and starts at zero, ``scaling = alpha / rank``, and the
unmerged forward is ``base(x) + B(A(dropout(x))) * scaling``.  The merge adds
``scaling * B @ A``, formed in fp32, into the base weight in its own dtype;
the unmerge subtracts the same product.
"""

from __future__ import annotations

import math
from collections.abc import Iterable

import torch


class LoraLinear(torch.nn.Module):
    def __init__(self, base: torch.nn.Linear, rank: int, alpha: float, *, dropout: float = 0.0,
                 adapter: str = "default", adapter_dtype: torch.dtype = torch.float32):
        super().__init__()
        if base.bias is not None:
            raise ValueError("LoraLinear wraps bias-free linears")
        self.base_layer = base
        dev = base.weight.device
        a = torch.nn.Linear(base.in_features, rank, bias=False, device=dev, dtype=adapter_dtype)
        b = torch.nn.Linear(rank, base.out_features, bias=False, device=dev, dtype=adapter_dtype)
        torch.nn.init.kaiming_uniform_(a.weight, a=math.sqrt(5))
        torch.nn.init.zeros_(b.weight)
        self.lora_A = torch.nn.ModuleDict({adapter: a})
        self.lora_B = torch.nn.ModuleDict({adapter: b})
        self.lora_dropout = torch.nn.ModuleDict(
            {adapter: torch.nn.Dropout(dropout) if dropout else torch.nn.Identity()})
        self.scaling = {adapter: alpha / rank}
        self.merged_adapters: list[str] = []

    def _delta(self, adapter: str) -> torch.Tensor:
        b, a = self.lora_B[adapter].weight, self.lora_A[adapter].weight
        return (b.detach().float() @ a.detach().float()) * self.scaling[adapter]

    @torch.no_grad()
    def merge(self, adapter_names: Iterable[str] | None = None) -> None:
        for name in adapter_names or list(self.lora_A):
            if name in self.merged_adapters:
                continue
            w = self.base_layer.weight
            w.copy_((w.float() + self._delta(name)).to(w.dtype))
            self.merged_adapters.append(name)

    @torch.no_grad()
    def unmerge(self) -> None:
        while self.merged_adapters:
            name = self.merged_adapters.pop()
            w = self.base_layer.weight
            w.copy_((w.float() - self._delta(name)).to(w.dtype))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self.base_layer(x)
        if self.merged_adapters:
            return y
        for name in self.lora_A:
            a, b = self.lora_A[name], self.lora_B[name]
            h = self.lora_dropout[name](x).to(a.weight.dtype)
            y = y + (b(a(h)) * self.scaling[name]).to(y.dtype)
        return y


def add_lora(model: torch.nn.Module, targets: Iterable[str], rank: int, alpha: float, *, dropout: float = 0.0,
             adapter_dtype: torch.dtype = torch.float32) -> int:
    """Wrap every ``nn.Linear`` whose attribute name is in ``targets`` (e.g.
    ``q_proj``) in a :class:`LoraLinear`, freeze everything but the adapters,
    and set ``model.active_adapter``; returns the number of layers wrapped."""
    names = set(targets)
    wrapped = 0
    for p in model.parameters():
        p.requires_grad_(False)
    for parent in list(model.modules()):
        for attr, child in list(parent.named_children()):
            if attr in names and isinstance(child, torch.nn.Linear):
                setattr(parent, attr, LoraLinear(child, rank, alpha, dropout=dropout, adapter_dtype=adapter_dtype))
                wrapped += 1
    model.active_adapter = "default"
    return wrapped
