"""Host-side contract of the merged-weight LoRA path (CPU: nothing launches).

Mirrors the reference's gates (tests/test_fused_lora.py): fusing merges the
adapter into the base weight and converts every eligible layer; unfusing
restores the stock forward and the base weight; a layer with active dropout
is declined; more than one active adapter is refused.  The fused forward
itself is GPU-only and refuses CPU tensors.  These CPU layers are ones the
kernels would not take (tests/test_fused_lora_host.py), so the tests of the
merge mechanics stand in an eligibility test that accepts them.
"""

from __future__ import annotations

import pytest
import torch

from thundersync_amd import fused_lora
from thundersync_amd.lora_layers import LoraLinear, add_lora


def _model(seed, dropout=0.0):
    torch.manual_seed(seed)
    base = torch.nn.Sequential()
    base.add_module("up", torch.nn.Linear(64, 128, bias=False))
    base.add_module("act", torch.nn.Tanh())
    base.add_module("down", torch.nn.Linear(128, 64, bias=False))
    assert add_lora(base, ["up", "down"], rank=8, alpha=16, dropout=dropout) == 2
    for layer in base.modules():
        if isinstance(layer, LoraLinear):
            torch.nn.init.normal_(layer.lora_B["default"].weight, std=0.1)
    return base


@pytest.fixture
def eligible(monkeypatch):
    monkeypatch.setattr(fused_lora, "fusable", lambda base, a, b: True)


def test_fuse_merges_and_unfuse_restores(eligible):
    model = _model(13)
    x = torch.randn(16, 64)
    before = model(x).detach().clone()
    w0 = model.up.base_layer.weight.detach().clone()
    a, b = model.up.lora_A["default"].weight.detach(), model.up.lora_B["default"].weight.detach()
    assert fused_lora.fuse_merged_lora_forward(model) == 2
    torch.testing.assert_close(model.up.base_layer.weight, w0 + 2.0 * b @ a, rtol=1e-5, atol=1e-6)
    assert model.up._thundersync_fused and model.down._thundersync_fused
    assert fused_lora.fuse_merged_lora_forward(model) == 0  # already fused
    assert fused_lora.unfuse_merged_lora_forward(model) == 2
    torch.testing.assert_close(model.up.base_layer.weight, w0, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(model(x), before, rtol=1e-5, atol=1e-6)
    assert not model.up._thundersync_fused and not hasattr(model.up, "_thundersync_unfused_forward")


def test_merged_module_forward_matches_the_unmerged_one():
    model = _model(3)
    x = torch.randn(9, 64)
    unmerged = model(x).detach()
    for layer in (model.up, model.down):
        layer.merge(adapter_names=["default"])
    torch.testing.assert_close(model(x), unmerged, rtol=1e-5, atol=1e-5)


def test_fusion_declines_a_layer_with_active_dropout(eligible):
    assert fused_lora.fuse_merged_lora_forward(_model(17, dropout=0.1)) == 0


def test_more_than_one_active_adapter_is_refused(eligible):
    model = _model(5)
    model.active_adapter = ["default", "other"]
    with pytest.raises(ValueError, match="one active adapter"):
        fused_lora.fuse_merged_lora_forward(model)


def test_fused_forward_refuses_cpu_tensors(eligible):
    model = _model(7)
    assert fused_lora.fuse_merged_lora_forward(model) == 2
    with pytest.raises(RuntimeError, match="GPU only"):
        model(torch.randn(4, 64))
