"""``forest_attention`` (engine/attention.py:186-231 of the reference) on the GPU
against the CPU oracle.

* Random segment forests -- shared prompts, trajectories that share their
  first turns, several levels -- on the physical stream: the HIP output and
  the gradients of Q, K and V against fp32 attention under the dense
  visibility mask that the oracle's own forest builder produces
  (``kv <= q < subtree_end[kv]``, engine/plan.py:343-362), with autograd.
* The C2 bench forest at full size (seed 0: 2048-token prompt, 8
  completions, 21,810 tokens, 32/8 heads) in one launch per direction; the
  prompt's rows and two completions checked against the oracle run on their
  own paths: outputs, dQ, and the dK/dV of a completion's own keys (read by
  that completion alone); and the shared prompt's dK/dV for KV head 0 in
  full -- its 2048 keys summed over every row of the forest that reads them
  (the prompt's own causal rows and all eight completions, 21,810 rows x 4
  query heads).

Bar: 2e-2 max-abs, scaled by max|ref| where that exceeds 1 (as for the other
attention tests).
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle import attention as ref
from oracle import forest as ofo
from thundersync_amd import attention as hip
from thundersync_amd import forest as prod

pytestmark = pytest.mark.gpu

D = 128


def close(got, want, what, bar=2e-2):
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = (got - want).abs().max().item() if got.numel() else 0.0
    scale = max(1.0, want.abs().max().item() if want.numel() else 0.0)
    print(f"    {what}: max-abs {err:.4g} (bar {bar * scale:.4g} = {bar} x max(1, max|ref| {scale:.3g}))", flush=True)
    assert err <= bar * scale, f"{what}: max-abs {err:.4g} > {bar} x {scale:.3g}"
    return err


def random_spec(seed, groups, per_group, prompt, first_turn, turns):
    """Trajectories as (group, id, [(kind, tokens, scored)]); within a group
    every trajectory repeats the prompt, and half of them also repeat the
    group's first action, so the forest has shared nodes below the roots."""
    rng = random.Random(seed)
    spec, tid = [], 0
    for g in range(groups):
        p = [rng.randrange(50000) for _ in range(rng.randint(*prompt))]
        shared = [rng.randrange(50000) for _ in range(rng.randint(*first_turn))]
        for i in range(per_group):
            segs = [("prompt", p, False)]
            if i % 2 == 0:
                segs.append(("action", shared, True))
            for _ in range(rng.randint(1, turns)):
                segs.append(("action", [50000 + tid] + [rng.randrange(50000) for _ in range(rng.randint(*first_turn))],
                             True))
                if rng.random() < 0.6:
                    segs.append(("observation", [rng.randrange(50000) for _ in range(rng.randint(1, 40))], False))
            spec.append((g, tid, segs))
            tid += 1
    return spec


def plans(spec):
    kinds = {"prompt": prod.SegmentKind.PROMPT, "action": prod.SegmentKind.ACTION,
             "observation": prod.SegmentKind.OBSERVATION}
    p_trajs = [prod.Trajectory([prod.Segment(tuple(t), kinds[k], s) for k, t, s in segs], group_id=g, traj_id=i)
               for g, i, segs in spec]
    o_trajs = [ofo.Trajectory([ofo.Segment(tuple(t), k, s) for k, t, s in segs], g, i) for g, i, segs in spec]
    return prod.compile_plan(prod.build_forest(p_trajs)), ofo.compile_plan(ofo.build_forest(o_trajs))


FORESTS = [
    # seed, groups, per_group, prompt lengths, turn lengths, turns, hq, hkv
    (0, 1, 3, (40, 60), (5, 20), 2, 8, 2),
    (1, 2, 4, (100, 200), (20, 90), 3, 32, 8),
    (2, 3, 3, (1, 8), (1, 6), 4, 4, 1),
    (3, 1, 6, (300, 300), (60, 130), 2, 40, 8),
]


@pytest.mark.parametrize("seed,groups,per_group,prompt,turn,turns,hq,hkv", FORESTS)
def test_forest_matches_masked_oracle(cuda, seed, groups, per_group, prompt, turn, turns, hq, hkv):
    spec = random_spec(seed, groups, per_group, prompt, turn, turns)
    plan, oplan = plans(spec)
    p = plan.n_physical
    print(f"forest seed {seed}: {p} tokens, {plan.n_nodes} nodes, depth {int(plan.node_depth.max())}, "
          f"{hq}/{hkv} heads", flush=True)
    mask = torch.tensor(ofo.visibility_mask(oplan))
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(p, hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(p, hkv, D, generator=g).to(torch.bfloat16)
    v = torch.randn(p, hkv, D, generator=g).to(torch.bfloat16)
    dout = torch.randn(p, hq, D, generator=g).to(torch.bfloat16)
    scale = D ** -0.5

    qd, kd, vd = (t.to(cuda).requires_grad_() for t in (q, k, v))
    out = hip.forest_attention(qd, kd, vd, plan.to(cuda), scale=scale)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()

    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    want = ref.masked_attention(qf, kf, vf, mask, scale)
    want.backward(dout.float())
    close(out, want, "out")
    close(qd.grad, qf.grad, "dq")
    close(kd.grad, kf.grad, "dk")
    close(vd.grad, vf.grad, "dv")


def test_c2_full_size_sampled(cuda):
    import bench

    print("C2 full size, seed 0", flush=True)
    plan, lengths, q, k, v, dout = bench.c2_inputs(0, cuda)
    scale = D ** -0.5
    out = hip.forest_attention(q, k, v, plan.to(cuda), scale=scale)
    out.backward(dout)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(q.grad).all()
    assert torch.isfinite(k.grad).all() and torch.isfinite(v.grad).all()
    starts, ends = plan.node_start.tolist(), plan.node_end.tolist()
    assert plan.n_nodes == 9 and (starts[0], ends[0]) == (0, 2048)

    qc, kc, vc, dc = (t.detach().cpu() for t in (q, k, v, dout))
    # the prompt's rows see the prompt alone
    o, gq, _, _ = ref.attention_with_grads(qc[:2048], [kc[:2048]], [vc[:2048]], dc[:2048], scale)
    print(f"  prompt: 2048 rows", flush=True)
    close(out[:2048], o, "out[prompt]")
    # the prompt's dQ also needs only its own rows' softmax
    close(q.grad[:2048], gq, "dq[prompt]")
    # the shortest and the longest completion: prompt keys, then their own
    by_len = sorted(range(1, 9), key=lambda n: ends[n] - starts[n])
    for n in (by_len[0], by_len[-1]):
        s, e = starts[n], ends[n]
        print(f"  completion node {n}: {e - s} rows over {2048 + e - s} keys", flush=True)
        o, gq, gk, gv = ref.attention_with_grads(qc[s:e], [kc[:2048], kc[s:e]], [vc[:2048], vc[s:e]], dc[s:e],
                                                 scale)
        close(out[s:e], o, f"out[node {n}]")
        close(q.grad[s:e], gq, f"dq[node {n}]")
        close(k.grad[s:e], gk[1], f"dk[node {n}]")
        close(v.grad[s:e], gv[1], f"dv[node {n}]")

    # the shared prompt's keys, KV head 0 (query heads 0-3): every node's rows read them
    want_dk = torch.zeros(2048, 1, D)
    want_dv = torch.zeros(2048, 1, D)
    for n in range(9):
        s, e = starts[n], ends[n]
        ks = [kc[:2048, :1]] if n == 0 else [kc[:2048, :1], kc[s:e, :1]]
        vs = [vc[:2048, :1]] if n == 0 else [vc[:2048, :1], vc[s:e, :1]]
        dk, dv = ref.prefix_key_grads(qc[s:e, :4], ks, vs, dc[s:e, :4], scale, 2048)
        want_dk += dk
        want_dv += dv
    print(f"  shared prompt dK/dV, KV head 0: {ends[8] - starts[0]} rows", flush=True)
    close(k.grad[:2048, :1], want_dk, "dk[prompt, kv head 0]")
    close(v.grad[:2048, :1], want_dv, "dv[prompt, kv head 0]")
