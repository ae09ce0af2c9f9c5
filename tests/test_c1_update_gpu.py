"""Config C1 through the device path: one GRPO-shaped update of the tiny
random-init Qwen3-style decoder (2 layers, hidden 128, 4 query / 2 KV heads,
head dim 32, SwiGLU MLP 384, vocab 1024, weights N(0, 0.02) from the seed) on
one prompt group of 4 trajectories sharing a 32-token prompt, completions
uniform in [8, 48], rewards N(0, 1) normalised by the group's population std.

The reference runs C1 in fp32 on the CPU; the build's kernels take bf16 or
fp16, so the update runs a bf16 copy of the same (bf16-representable)
weights on the GPU -- every parameter trainable, the forest attention adapter
over one pass of the group's forest, the HIP RMSNorm modules (hidden and
q/k norms), the fused logprob with its weight gradient (the head is
trainable) -- and is checked against the fp32 model on the CPU with its stock
eager attention, trajectory by trajectory: the reward-linear loss, every
parameter's gradient and one SGD step.  Bars: the loss within 1e-2 relative;
gradients and updated-minus-initial weights within 5e-2 relative Frobenius
error (bf16 weights and activations through two layers, forward and
backward, against fp32; measured below 2e-2)."""

from __future__ import annotations

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")


def c1_model(seed: int):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config(vocab_size=1024, hidden_size=128, intermediate_size=384, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=32, tie_word_embeddings=False,
                      initializer_range=0.02, attn_implementation="eager")
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(cfg).float()
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(p.to(torch.bfloat16).float())  # both copies hold the same bf16 values
    return model


def c1_rollouts(seed: int):
    g = torch.Generator().manual_seed(seed)
    prompt = torch.randint(0, 1024, (32,), generator=g).tolist()
    lengths = torch.randint(8, 49, (4,), generator=g).tolist()
    bodies = [torch.randint(0, 1024, (n,), generator=g).tolist() for n in lengths]
    rewards = torch.randn(4, generator=g)
    adv = (rewards - rewards.mean()) / rewards.std(unbiased=False)
    return prompt, bodies, adv


def rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_c1_grpo_update(cuda):
    from thundersync_amd import forest
    from thundersync_amd.attention import HIP_FOREST_ATTENTION_NAME, forest_context, register_attention
    from thundersync_amd.rms_norm import use_stable_qwen3_rms_norm
    from thundersync_amd.step import forest_logprobs, split_by_trajectory

    print("C1: tiny Qwen3 GRPO update through the build vs the fp32 CPU model", flush=True)
    assert register_attention()
    ref = c1_model(seed=0)
    prompt, bodies, adv = c1_rollouts(seed=1)
    print(f"  completions {[len(b) for b in bodies]}, advantages {[round(a, 3) for a in adv.tolist()]}", flush=True)
    gpu = copy.deepcopy(ref).to(device=cuda, dtype=torch.bfloat16)
    gpu.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)
    assert use_stable_qwen3_rms_norm(gpu) == 2 * 4 + 1  # per layer: input, post-attention, q and k norms; the final norm
    gpu.train()

    trajs = [forest.Trajectory([forest.Segment.prompt(prompt), forest.Segment.action(b)], group_id=0, traj_id=i)
             for i, b in enumerate(bodies)]
    plan = forest.compile_plan(forest.build_forest(trajs)).to(cuda)
    n_tokens = sum(len(b) for b in bodies)
    with forest_context(plan):
        lp = forest_logprobs(gpu, plan)
        per = split_by_trajectory(plan, lp)
        loss = -sum(float(adv[t]) * v.float().sum() for t, v in per.items()) / n_tokens
        loss.backward()
    torch.cuda.synchronize()
    assert lp.numel() == n_tokens

    want = torch.zeros(())
    for i, body in enumerate(bodies):
        tokens = torch.tensor(prompt + body)
        logits = ref(input_ids=tokens[None]).logits[0]
        lp_i = torch.log_softmax(logits, -1)[len(prompt) - 1 : -1].gather(1, tokens[len(prompt):, None])[:, 0]
        want = want - float(adv[i]) * lp_i.sum() / n_tokens
    want.backward()
    err = abs(loss.item() - want.item()) / abs(want.item())
    print(f"  loss {loss.item():.6f} vs {want.item():.6f} (relative {err:.2e})", flush=True)
    assert err < 1e-2

    got = {n: p for n, p in gpu.named_parameters()}
    exp = {n: p for n, p in ref.named_parameters()}
    assert set(got) == set(exp)
    worst = 0.0
    for name in sorted(exp):
        assert got[name].grad is not None and exp[name].grad is not None, name
        e = rel(got[name].grad, exp[name].grad)
        worst = max(worst, e)
        assert e < 5e-2, (name, e)
    print(f"  {len(exp)} parameter gradients: worst relative error {worst:.2e}", flush=True)

    # one SGD update on both; the GPU copy's step is taken in fp32 from its
    # bf16 gradients so that the comparison sees the gradients, not bf16 steps
    lr = 0.5
    worst = 0.0
    for name in sorted(exp):
        before = exp[name].detach().clone()
        with torch.no_grad():
            exp[name] -= lr * exp[name].grad
            step_gpu = -lr * got[name].grad.float()
        e = rel(step_gpu, exp[name].detach() - before)
        worst = max(worst, e)
        assert e < 5e-2, (name, e)
    print(f"  SGD update of {len(exp)} parameters: worst relative error {worst:.2e}", flush=True)


def test_c1_grpo_update_in_fp32(cuda):
    """C1 at its stated precision: the fp32 model on the GPU, each
    trajectory's hidden states from the stock decoder (attention through
    torch's SDPA, which is where the reference's dispatch sends fp32
    attention: its flash kernels take bf16 / fp16 only) and every scored
    token's logprob through the fused logprob's fp32 kernels with the
    trainable head; against the fp32 model on the CPU.  Bars: loss within
    1e-5 relative, every gradient within 1e-4 relative Frobenius error (fp32
    against fp32; only summation orders differ)."""
    from thundersync_amd.fused_logprob import fused_logprob

    print("C1 in fp32: tiny Qwen3 GRPO update, fused fp32 logprob on the GPU vs the fp32 CPU model", flush=True)
    ref = c1_model(seed=0)
    prompt, bodies, adv = c1_rollouts(seed=1)
    gpu = copy.deepcopy(ref).to(device=cuda)
    gpu.config._attn_implementation = "sdpa"
    gpu.train()
    n_tokens = sum(len(b) for b in bodies)
    loss = torch.zeros((), device=cuda)
    for i, body in enumerate(bodies):
        tokens = torch.tensor(prompt + body, device=cuda)
        hidden = gpu.model(input_ids=tokens[None]).last_hidden_state[0]
        rows = hidden[len(prompt) - 1 : -1]
        lp = fused_logprob(rows, gpu.lm_head.weight, tokens[len(prompt):], chunk=16)
        assert lp.dtype == torch.float32
        loss = loss - float(adv[i]) * lp.sum() / n_tokens
    loss.backward()
    torch.cuda.synchronize()

    want = torch.zeros(())
    for i, body in enumerate(bodies):
        tokens = torch.tensor(prompt + body)
        logits = ref(input_ids=tokens[None]).logits[0]
        lp_i = torch.log_softmax(logits, -1)[len(prompt) - 1 : -1].gather(1, tokens[len(prompt):, None])[:, 0]
        want = want - float(adv[i]) * lp_i.sum() / n_tokens
    want.backward()
    err = abs(loss.item() - want.item()) / abs(want.item())
    print(f"  loss {loss.item():.8f} vs {want.item():.8f} (relative {err:.2e})", flush=True)
    assert err < 1e-5

    got = {n: p for n, p in gpu.named_parameters()}
    exp = {n: p for n, p in ref.named_parameters()}
    worst = 0.0
    for name in sorted(exp):
        if exp[name].grad is None:  # the input embedding of unused tokens aside, every parameter learns
            assert got[name].grad is None, name
            continue
        e = rel(got[name].grad, exp[name].grad)
        worst = max(worst, e)
        assert e < 1e-4, (name, e)
    print(f"  parameter gradients: worst relative error {worst:.2e}", flush=True)
