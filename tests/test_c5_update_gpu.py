"""One GRPO-shaped update at the C5 config's shapes.

Two layers of the Qwen3-8B-shaped decoder (hidden 4096, 32 query / 8 KV
heads, head dim 128, MLP 12288, vocab 151936, random-init bf16) with LoRA
rank 16 on q/k/v/o (fp32 adapters, merged-weight path), the HIP RMSNorm
modules, the forest attention adapter, per-layer activation checkpointing
and the fused head, over the C5 rollouts (2 groups x 8 trajectories,
1024-token prompts, completions U[512, 8192]; 88,105 physical tokens with
seed 0).  One reward-linear update, then:

* every logprob and every adapter gradient is finite, and the training
  pass's logprobs equal a no-grad pass's bit for bit (same kernels, the
  checkpoint recompute included);
* two sampled trajectories (one per group) through the same bf16 model run
  alone with the causal adapter: only the packing differs; bar 2e-2 nat
  (|log p| ~ 12 for a random 151936-way head; bf16 attention outputs differ
  in the last bit between the two packings and travel through two layers);
* layer 0's q_proj adapter gradients against the fp64 oracle of the fused
  backward (accel/fused_lora.py:35-48) on the layer's own captured input and
  output gradient, with the rank products rounded to bf16 as the device
  forms them; bar 2e-3 x max|oracle| (as tests/test_lora_gpu.py).
"""

from __future__ import annotations

import pytest
import torch

from oracle import lora as lora_ref

pytestmark = pytest.mark.gpu

transformers = pytest.importorskip("transformers")

VOCAB, HIDDEN, MLP, HQ, HKV, D = 151936, 4096, 12288, 32, 8, 128


def c5_model(device, layers=2):
    from transformers import Qwen3Config, Qwen3ForCausalLM

    from thundersync_amd.attention import HIP_FOREST_ATTENTION_NAME, register_attention
    from thundersync_amd.lora_layers import add_lora
    from thundersync_amd.rms_norm import use_stable_qwen3_rms_norm

    cfg = Qwen3Config(vocab_size=VOCAB, hidden_size=HIDDEN, intermediate_size=MLP, num_hidden_layers=layers,
                      num_attention_heads=HQ, num_key_value_heads=HKV, head_dim=D, tie_word_embeddings=False,
                      max_position_embeddings=40960, rms_norm_eps=1e-6)
    torch.manual_seed(0)
    default = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen3ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(default)
    assert register_attention()
    model.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)
    use_stable_qwen3_rms_norm(model)
    assert add_lora(model, ["q_proj", "k_proj", "v_proj", "o_proj"], rank=16, alpha=32) == 4 * layers
    g = torch.Generator(device=device).manual_seed(1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if "lora_B" in name:  # B starts at zero; give the adapters a gradient path through both
                p.copy_(torch.randn(p.shape, generator=g, device=device) * 0.02)
    model.gradient_checkpointing_enable(gradient_checkpointing_kwargs={"use_reentrant": False})
    model.train()
    return model


def c5_rollouts(seed=0):
    """The C5 rollouts: 2 groups x 8 trajectories, prompt 1024, completions
    U[512, 8192], uniform tokens; group-std-normalised advantages."""
    from thundersync_amd import forest

    g = torch.Generator().manual_seed(seed)
    trajs, rewards, tokens = [], [], {}
    for grp in range(2):
        prompt = torch.randint(0, VOCAB, (1024,), generator=g).tolist()
        lengths = torch.randint(512, 8193, (8,), generator=g).tolist()
        for i, n in enumerate(lengths):
            body = torch.randint(0, VOCAB, (n,), generator=g).tolist()
            tid = 8 * grp + i
            tokens[tid] = (prompt, body)
            trajs.append(forest.Trajectory([forest.Segment.prompt(prompt), forest.Segment.action(body)],
                                           group_id=grp, traj_id=tid))
        rewards.append(torch.randn(8, generator=g))
    r = torch.stack(rewards)
    adv = ((r - r.mean(1, keepdim=True)) / r.std(1, unbiased=False, keepdim=True).clamp_min(1e-6)).flatten()
    return trajs, {i: float(adv[i]) for i in range(16)}, tokens


def test_c5_update_at_full_shape(cuda):
    from thundersync_amd import forest
    from thundersync_amd.attention import HIP_ATTENTION_NAME, HIP_FOREST_ATTENTION_NAME, forest_context
    from thundersync_amd.fused_logprob import fused_logprob
    from thundersync_amd.fused_lora import fuse_merged_lora_forward, unfuse_merged_lora_forward
    from thundersync_amd.step import forest_logprobs, split_by_trajectory, unembedding

    print("C5 update: building 2 layers of the C5 decoder and the C5 forest", flush=True)
    model = c5_model(cuda)
    trajs, adv, tokens = c5_rollouts()
    plan = forest.compile_plan(forest.build_forest(trajs)).to(cuda)
    assert plan.n_physical == 1024 * 2 + sum(len(b) for _, b in tokens.values())
    q_proj = model.model.layers[0].self_attn.q_proj
    captured = {}

    def keep_input(module, args, output):
        captured["x"] = args[0].detach()
        if output.requires_grad:
            output.register_hook(lambda grad: captured.__setitem__("g", grad.detach()))

    handle = q_proj.register_forward_hook(keep_input)
    print(f"C5 update: one update over {plan.n_physical} tokens", flush=True)
    assert fuse_merged_lora_forward(model) == 8
    with forest_context(plan):
        lp = forest_logprobs(model, plan)
        per = split_by_trajectory(plan, lp)
        loss = -sum(adv[tid] * v.sum() for tid, v in per.items()) / lp.numel()
        loss.backward()
    torch.cuda.synchronize()
    handle.remove()
    assert lp.numel() == int(plan.score_src.numel()) == sum(len(b) for _, b in tokens.values())
    assert bool(lp.isfinite().all()) and bool((lp <= 0).all())
    grads = {n: p.grad for n, p in model.named_parameters() if p.grad is not None}
    assert len(grads) == 16 and all("lora_" in n for n in grads)
    for name, grad in grads.items():
        assert grad.dtype == torch.float32 and bool(grad.isfinite().all()), name
        assert float(grad.abs().max()) > 0, name

    print("C5 update: no-grad forest pass and two trajectories alone", flush=True)
    with torch.no_grad():
        with forest_context(plan):
            lp_eval = forest_logprobs(model, plan)
        assert torch.equal(lp_eval, lp.detach())
        per_eval = split_by_trajectory(plan, lp_eval)
        model.set_attn_implementation(HIP_ATTENTION_NAME)
        try:
            for tid in (0, 9):
                prompt, body = tokens[tid]
                ids = torch.tensor(prompt + body, device=cuda)
                hidden = model.model(input_ids=ids[None]).last_hidden_state[0]
                alone = fused_logprob(hidden[len(prompt) - 1: -1], unembedding(model), ids[len(prompt):])
                err = (per_eval[tid] - alone).abs().max().item()
                print(f"  trajectory {tid} ({len(body)} tokens): forest vs alone max |diff| {err:.3e}", flush=True)
                assert err < 2e-2, (tid, err)
        finally:
            model.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)
    assert unfuse_merged_lora_forward(model) == 8

    print("C5 update: layer 0 q_proj adapter gradients against the oracle", flush=True)
    a = q_proj.lora_A["default"].weight
    b = q_proj.lora_B["default"].weight
    x = captured["x"].reshape(-1, HIDDEN).cpu()
    g = captured["g"].reshape(-1, HQ * D).cpu()
    _, want_da, want_db = lora_ref.fused_backward(g, x, None, a.detach().to(torch.bfloat16).cpu(),
                                                  b.detach().to(torch.bfloat16).cpu(), q_proj.scaling["default"],
                                                  round_rank=True)
    for what, got, want in (("dA", a.grad, want_da), ("dB", b.grad, want_db)):
        got = got.double().cpu()
        err = (got - want).abs().max().item()
        scale = want.abs().max().item()
        print(f"  {what}: max-abs {err:.3g} (bar 2e-3 x {scale:.3g})", flush=True)
        assert err <= 2e-3 * scale, what
