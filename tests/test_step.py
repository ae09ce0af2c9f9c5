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


def test_assert_supported_refuses_recurrent_layers():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from thundersync_amd.step import assert_supported

    cfg = Qwen3Config(vocab_size=32, hidden_size=64, intermediate_size=96, num_hidden_layers=2,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=32)
    model = Qwen3ForCausalLM(cfg)
    assert_supported(model)  # plain attention stack: accepted (and memoised)
    assert_supported(model)
    hybrid = Qwen3ForCausalLM(cfg)
    hybrid.config.layer_types = ["full_attention", "linear_attention"]
    with pytest.raises(NotImplementedError, match="non-attention layer types"):
        assert_supported(hybrid)

    class MambaMixer(torch.nn.Module):
        pass

    recurrent = Qwen3ForCausalLM(cfg)
    recurrent.model.layers[0].extra = MambaMixer()
    with pytest.raises(NotImplementedError, match="recurrent state"):
        assert_supported(recurrent)


def test_forest_logprobs_stats_without_a_device(monkeypatch):
    """The gated and ungated projections and their accounting, with the
    hidden states and the fused projection stood in for on the CPU."""
    from thundersync_amd import step

    trajs = [forest.Trajectory([forest.Segment.prompt([1, 2, 3]), forest.Segment.action(body)], group_id=0, traj_id=t)
             for t, body in enumerate(([4, 5, 6], [4, 5, 7, 8], [9]))]
    plan = forest.compile_plan(forest.build_forest(trajs))
    calls = []

    def fake_fused(h, w, t, chunk=1024):
        calls.append(int(h.shape[0]))
        return (h[:, 0] * 1000 + t).float()  # identifies (source row, target)

    monkeypatch.setattr(step, "fused_logprob", fake_fused)
    monkeypatch.setattr(step, "forest_context", lambda plan: __import__("contextlib").nullcontext())
    hidden = torch.arange(plan.n_physical, dtype=torch.float32)[:, None].repeat(1, 4)
    model = torch.nn.Linear(4, 4)
    gated, stats = step.forest_logprobs(model, plan, weight=torch.zeros(16, 4), hidden_fn=lambda i, p: hidden,
                                        return_stats=True)
    ungated = step.forest_logprobs(model, plan, weight=torch.zeros(16, 4), hidden_fn=lambda i, p: hidden, gate=False)
    assert torch.equal(gated, ungated)
    want = (plan.score_src.float() * 1000 + plan.score_tgt.float()).index_select(0, plan.logical_to_slot)
    assert torch.equal(gated, want)
    assert stats.physical_tokens == plan.n_physical and stats.logical_tokens == 3 * 3 + 3 + 4 + 1
    assert stats.padded_tokens == 3 * 7 and stats.projected_positions == plan.score_src.numel()
    assert calls[0] == plan.score_src.numel() and calls[1] == plan.n_physical


def test_step_stats_ratios_and_text():
    """engine/step.py:170-194: both ratios are against the padded rectangle."""
    from thundersync_amd.step import StepStats

    stats = StepStats(physical_tokens=10, logical_tokens=16, padded_tokens=21, projected_positions=7,
                      logical_scored=8)
    assert stats.token_compression == 21 / 10
    assert stats.projection_reduction == 21 / 7
    assert str(stats) == "tokens 21 -> 10 (2.10x)   projected 21 -> 7 (3.00x)"
    assert StepStats(0, 0, 0, 0, 0).token_compression == 0.0


def test_split_by_trajectory_concatenates_a_repeated_id():
    """Trajectory ids default to 0 and need not be unique: every token of an
    id is returned, in logical order, as the reference's mask selection does
    (engine/step.py:483-486)."""
    trajs = [forest.Trajectory([forest.Segment.prompt([1, 2, 3]), forest.Segment.action(body)], group_id=0,
                               traj_id=t)
             for t, body in zip((0, 1, 0), ([4, 5, 6], [4, 5, 7, 8], [9]))]
    plan = forest.compile_plan(forest.build_forest(trajs))
    logical = torch.arange(plan.logical_to_slot.numel(), dtype=torch.float32)
    per = split_by_trajectory(plan, logical)
    traj = plan.logical_traj
    # id 0 comes back after id 1: two separate runs of it in logical order
    assert torch.unique_consecutive(traj).tolist() == [0, 1, 0]
    assert sorted(per) == [0, 1]
    for tid in (0, 1):
        assert torch.equal(per[tid], logical[traj == tid])
