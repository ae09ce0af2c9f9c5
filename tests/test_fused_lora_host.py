"""fuse_merged_lora_forward's eligibility test (host logic, CPU).

Layers the kernels cannot run -- CPU or fp32 base weights, features that are
not multiples of 8, ranks above the kernels' limit -- must be left exactly as
they were: not merged (the base weight unchanged) and not rerouted, so they
keep running their own unmerged forward, as the reference's torch-matmul
FusedLoRALinear would run them (accel/fused_lora.py:29-48).
"""

from __future__ import annotations

import torch

from thundersync_amd import fused_lora
from thundersync_amd.lora_layers import LoraLinear, add_lora


def _model(inp, out, rank, dtype=torch.float32):
    torch.manual_seed(3)
    model = torch.nn.Sequential()
    model.add_module("proj", torch.nn.Linear(inp, out, bias=False, dtype=dtype))
    add_lora(model, ["proj"], rank=rank, alpha=2 * rank)
    layer = model.proj
    torch.nn.init.normal_(layer.lora_B["default"].weight, std=0.05)
    return model, layer


def _untouched(model, layer, inp, dtype=torch.float32):
    before = layer.base_layer.weight.detach().clone()
    x = torch.randn(5, inp).to(dtype)
    want = model(x)
    assert fused_lora.fuse_merged_lora_forward(model) == 0
    assert torch.equal(layer.base_layer.weight, before)
    assert not layer.merged_adapters
    assert not getattr(layer, fused_lora._FLAG, False)
    assert "forward" not in vars(layer)
    assert torch.equal(model(x), want)
    assert fused_lora.unfuse_merged_lora_forward(model) == 0


def test_cpu_fp32_layer_is_left_unmerged():
    model, layer = _model(64, 32, 4)
    _untouched(model, layer, 64)


def test_cpu_bf16_layer_is_left_unmerged():
    model, layer = _model(64, 32, 4, torch.bfloat16)
    _untouched(model, layer, 64, torch.bfloat16)


def test_fusable_rules_on_meta_shapes():
    """The shape rules alone (a CPU weight fails first, so they are checked
    on a layer whose device test is bypassed)."""

    class FakeWeight:
        def __init__(self, shape, dtype=torch.bfloat16):
            self.shape, self.dtype, self.is_cuda, self.device = torch.Size(shape), dtype, True, "cuda:0"

        def dim(self):
            return len(self.shape)

    class FakeLinear:
        def __init__(self, out_f, in_f, dtype=torch.bfloat16):
            self.weight = FakeWeight((out_f, in_f), dtype)

    def ok(out_f, in_f, rank, dtype=torch.bfloat16):
        return fused_lora.fusable(FakeLinear(out_f, in_f, dtype), FakeWeight((rank, in_f)),
                                  FakeWeight((out_f, rank)))

    lib_present = fused_lora._lib.library
    try:
        fused_lora._lib.library = lambda: object()
        assert ok(64, 32, 16)
        assert ok(64, 32, fused_lora.MAX_RANK)
        assert not ok(64, 32, fused_lora.MAX_RANK + 1)
        assert not ok(60, 32, 16)
        assert not ok(64, 36, 16)
        assert not ok(64, 32, 16, torch.float32)
        fused_lora._lib.library = lambda: None
        assert not ok(64, 32, 16)
    finally:
        fused_lora._lib.library = lib_present


def test_a_mixed_model_converts_only_what_the_kernels_run():
    model, layer = _model(64, 32, 4)
    assert isinstance(layer, LoraLinear)
    calls = []
    original = fused_lora.fusable
    try:
        fused_lora.fusable = lambda base, a, b: calls.append(tuple(base.weight.shape)) or False
        assert fused_lora.fuse_merged_lora_forward(model) == 0
    finally:
        fused_lora.fusable = original
    assert calls == [(32, 64)]
