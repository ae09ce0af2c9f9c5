"""Host logic of thundersync_amd.step (engine/step.py:358-490 of the reference)."""

from __future__ import annotations

import pytest
import torch

from thundersync_amd import forest
from thundersync_amd.step import base_model, split_by_trajectory, unembedding

transformers = pytest.importorskip("transformers")


def test_base_model_and_unembedding():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config(vocab_size=32, hidden_size=64, intermediate_size=96, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=32, tie_word_embeddings=False)
    model = Qwen3ForCausalLM(cfg)
    assert base_model(model) is model.model
    assert unembedding(model) is model.lm_head.weight
    assert base_model(model.model) is model.model  # a bare stack is its own base
    with pytest.raises(AttributeError):
        unembedding(torch.nn.Sequential(torch.nn.ReLU()))


def test_split_by_trajectory_keeps_each_trajectorys_order():
    trajs = [forest.Trajectory([forest.Segment.prompt([1, 2, 3]), forest.Segment.action(body)], group_id=0, traj_id=t)
             for t, body in enumerate(([4, 5, 6], [4, 5, 7, 8], [9]))]
    plan = forest.compile_plan(forest.build_forest(trajs))
    logical = torch.arange(plan.logical_to_slot.numel(), dtype=torch.float32)
    per = split_by_trajectory(plan, logical)
    assert sorted(per) == [0, 1, 2]
    assert [per[t].numel() for t in range(3)] == [3, 4, 1]
    # logical order is trajectory by trajectory, so each piece is a contiguous run
    assert torch.equal(torch.cat([per[t] for t in range(3)]), logical)
