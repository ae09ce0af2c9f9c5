"""The attention adapters inside a HuggingFace Qwen3 decoder.

* ``hip_attention_forward`` (the ``fa4_attention_forward`` contract,
  accel/fa4_attention.py:22-53 of the reference): a bf16 model on the GPU with
  the HIP attention against the same weights in fp32 on the CPU with the
  stock eager attention -- last hidden states and parameter gradients.
* ``forest_logprobs`` (engine/step.py:383-472): one pass over a forest's
  physical stream with ``forest_attention_forward`` and the fused logprob
  against each trajectory run on its own through the CPU model and a plain
  log-softmax.  Gated and ungated projection agree.

Bars: relative Frobenius error 3e-2 for hidden states and gradients (bf16
weights and activations through two layers against fp32); 2e-2 nat absolute
for log-probabilities of a near-uniform random model (|log p| ~ 5) against the
fp32 CPU model (measured: under 5e-3), and 5e-3 nat against the same bf16 model
run on each trajectory alone, where only the packing differs (measured: 0).
"""

from __future__ import annotations

import copy

import pytest
import torch

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

HQ, HKV, D = 4, 1, 128


def tiny_model(seed=0):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config(vocab_size=96, hidden_size=256, intermediate_size=384, num_hidden_layers=2,
                      num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D, tie_word_embeddings=False,
                      attn_implementation="eager")
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(cfg).float()
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(p.to(torch.bfloat16).float())  # both copies hold the same bf16 values
    return model


def rel(a, b):
    a, b = a.detach().float().cpu(), b.detach().float().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_causal_adapter_in_model(cuda):
    from thundersync_amd.attention import HIP_ATTENTION_NAME, register_attention

    print("HF Qwen3 with the HIP causal adapter", flush=True)
    assert register_attention()
    ref = tiny_model()
    gpu = copy.deepcopy(ref).to(device=cuda, dtype=torch.bfloat16)
    gpu.set_attn_implementation(HIP_ATTENTION_NAME)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 96, (2, 77), generator=g)
    probe = torch.randn(2, 77, 256, generator=g)

    out_ref = ref.model(input_ids=ids).last_hidden_state
    (out_ref * probe).sum().backward()
    out = gpu.model(input_ids=ids.to(cuda)).last_hidden_state
    (out.float() * probe.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    assert rel(out, out_ref) < 3e-2
    for name in ("layers.0.self_attn.q_proj.weight", "layers.0.self_attn.k_proj.weight",
                 "layers.1.self_attn.v_proj.weight", "embed_tokens.weight"):
        a = dict(gpu.model.named_parameters())[name].grad
        b = dict(ref.model.named_parameters())[name].grad
        err = rel(a, b)
        print(f"  grad {name}: rel {err:.2e}", flush=True)
        assert err < 3e-2, name


def test_forest_logprobs_in_model(cuda):
    from thundersync_amd import forest
    from thundersync_amd.attention import HIP_FOREST_ATTENTION_NAME, register_attention
    from thundersync_amd.step import forest_logprobs, split_by_trajectory

    print("HF Qwen3 forest_logprobs over a shared-prompt forest", flush=True)
    assert register_attention()
    g = torch.Generator().manual_seed(2)
    prompt = torch.randint(0, 96, (40,), generator=g).tolist()
    shared = torch.randint(0, 96, (9,), generator=g).tolist()
    bodies = [shared + torch.randint(0, 96, (n,), generator=g).tolist() for n in (25, 31)]
    bodies.append(torch.randint(0, 96, (17,), generator=g).tolist())
    trajs = [forest.Trajectory([forest.Segment.prompt(prompt), forest.Segment.action(b)], group_id=0, traj_id=i)
             for i, b in enumerate(bodies)]
    plan = forest.compile_plan(forest.build_forest(trajs)).to(cuda)

    ref = tiny_model(seed=3)
    gpu = copy.deepcopy(ref).to(device=cuda, dtype=torch.bfloat16)
    gpu.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)
    with torch.no_grad():
        lp = forest_logprobs(gpu, plan)
        lp_all = forest_logprobs(gpu, plan, gate=False)
    torch.cuda.synchronize()
    torch.testing.assert_close(lp_all, lp, rtol=0, atol=1e-5)
    per = split_by_trajectory(plan, lp)
    assert sorted(per) == [0, 1, 2]
    for i, body in enumerate(bodies):
        tokens = torch.tensor(prompt + body)
        with torch.no_grad():
            logits = ref(input_ids=tokens[None]).logits[0]
        want = torch.log_softmax(logits, -1)[len(prompt) - 1 : -1].gather(1, tokens[len(prompt):, None])[:, 0]
        got = per[i].cpu()
        assert got.shape == want.shape, (i, got.shape, want.shape)
        err = (got - want).abs().max().item()
        print(f"  trajectory {i}: {got.numel()} scored tokens, max |diff| {err:.3e}", flush=True)
        assert err < 2e-2
    # the same bf16 model on the GPU, each trajectory alone through the causal
    # adapter and the fused head: only the packing differs, so the forest's
    # logprobs agree to the bf16 rounding of the attention outputs
    from thundersync_amd.attention import HIP_ATTENTION_NAME
    from thundersync_amd.fused_logprob import fused_logprob
    from thundersync_amd.step import unembedding

    gpu.set_attn_implementation(HIP_ATTENTION_NAME)
    for i, body in enumerate(bodies):
        ids = torch.tensor(prompt + body, device=cuda)
        with torch.no_grad():
            hidden = gpu.model(input_ids=ids[None]).last_hidden_state[0]
            alone = fused_logprob(hidden[len(prompt) - 1 : -1], unembedding(gpu), ids[len(prompt):])
        err = (per[i] - alone).abs().max().item()
        print(f"  trajectory {i}: forest vs alone (same bf16 model) max |diff| {err:.3e}", flush=True)
        assert err < 5e-3


def test_lora_grpo_update_through_the_build(cuda):
    """The C5 update's path at small scale: a bf16 Qwen3 with fp32 LoRA adapters
    on q/k/v/o, the forest attention adapter, the HIP RMSNorm modules, per-layer
    activation checkpointing, the merged-weight LoRA layers and the fused head,
    one reward-linear loss over a shared-prompt forest -- against the unmerged
    fp32 model on the CPU, trajectory by trajectory with its stock attention.
    Bars: the loss within 1e-2 relative, every adapter gradient within 3e-2
    relative Frobenius error (bf16 weights, merged weight and activations
    through two layers, forward and backward, against fp32)."""
    from thundersync_amd import forest
    from thundersync_amd.attention import HIP_FOREST_ATTENTION_NAME, forest_context, register_attention
    from thundersync_amd.fused_lora import fuse_merged_lora_forward, unfuse_merged_lora_forward
    from thundersync_amd.lora_layers import LoraLinear, add_lora
    from thundersync_amd.rms_norm import use_stable_qwen3_rms_norm
    from thundersync_amd.step import forest_logprobs, split_by_trajectory

    print("LoRA GRPO update through the build vs the unmerged fp32 model", flush=True)
    assert register_attention()
    ref = tiny_model(seed=5)
    assert add_lora(ref, ["q_proj", "k_proj", "v_proj", "o_proj"], rank=8, alpha=16) == 8
    g = torch.Generator().manual_seed(6)
    with torch.no_grad():
        for m in ref.modules():
            if isinstance(m, LoraLinear):
                for p in (m.lora_A["default"].weight, m.lora_B["default"].weight):
                    p.copy_((torch.randn(p.shape, generator=g) * 0.05).to(torch.bfloat16).float())
    gpu = copy.deepcopy(ref).to(device=cuda, dtype=torch.bfloat16)
    for m in gpu.modules():
        if isinstance(m, LoraLinear):
            m.lora_A.float()
            m.lora_B.float()
    gpu.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)
    use_stable_qwen3_rms_norm(gpu)
    gpu.gradient_checkpointing_enable(gradient_checkpointing_kwargs={"use_reentrant": False})
    gpu.train()

    prompt = torch.randint(0, 96, (40,), generator=g).tolist()
    bodies = [torch.randint(0, 96, (n,), generator=g).tolist() for n in (25, 31, 17)]
    adv = {0: 1.0, 1: -0.25, 2: -0.75}
    trajs = [forest.Trajectory([forest.Segment.prompt(prompt), forest.Segment.action(b)], group_id=0, traj_id=i)
             for i, b in enumerate(bodies)]
    plan = forest.compile_plan(forest.build_forest(trajs)).to(cuda)
    n_tokens = sum(len(b) for b in bodies)

    assert fuse_merged_lora_forward(gpu) == 8
    with forest_context(plan):
        lp = forest_logprobs(gpu, plan)
        per = split_by_trajectory(plan, lp)
        loss = -sum(adv[t] * v.sum() for t, v in per.items()) / lp.numel()
        loss.backward()
    torch.cuda.synchronize()
    assert unfuse_merged_lora_forward(gpu) == 8
    assert lp.numel() == n_tokens

    want = torch.zeros(())
    for i, body in enumerate(bodies):
        tokens = torch.tensor(prompt + body)
        logits = ref(input_ids=tokens[None]).logits[0]
        lp_i = torch.log_softmax(logits, -1)[len(prompt) - 1 : -1].gather(1, tokens[len(prompt):, None])[:, 0]
        want = want - adv[i] * lp_i.sum() / n_tokens
    want.backward()
    err = abs(loss.item() - want.item()) / abs(want.item())
    print(f"  loss {loss.item():.6f} vs {want.item():.6f} (relative {err:.2e})", flush=True)
    assert err < 1e-2
    got = {n: p.grad for n, p in gpu.named_parameters() if p.grad is not None}
    exp = {n: p.grad for n, p in ref.named_parameters() if p.grad is not None}
    assert set(got) == set(exp) and len(got) == 16
    worst = 0.0
    for name in sorted(exp):
        assert got[name].dtype == torch.float32, name
        e = rel(got[name], exp[name])
        worst = max(worst, e)
        assert e < 3e-2, (name, e)
    print(f"  16 adapter gradients: worst relative error {worst:.2e}", flush=True)
