"""HIP attention at head dims other than 128 against the CPU oracle.

The reference's attention paths take any head dim up to 256
(engine/streaming.py:532-548, :915-930); its own FA4 tests run D = 256 with
24 query heads on 4 KV heads (tests/test_fa4_bottom_right.py:13-28,
tests/test_fa4_attention.py:29-41).  Head dims 32, 64, 96, 192 and 256 run
the register-staged kernels (templated on the head dim; at 128 with GQA
groups that are a multiple of 4 the one-wave-per-head kernels run instead,
covered by the other attention tests), with every GQA group size: groups of
4 and 8 there take 48-key dK/dV work items like the 128 kernels, the others
64.  Bar as for the other attention tests: 2e-2 max-abs of the fp32 oracle,
scaled by max|ref| where that exceeds 1.
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as ref
from oracle import forest as ofo
from thundersync_amd import attention as hip
from thundersync_amd import forest as prod

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, params=["kv64", "kv48"])
def head_dim_256_items(request, monkeypatch):
    """Head dim 256 runs both dK/dV work-item sizes: the 64-key items of the
    two-waves-of-32-keys kernel (forced for these small shapes) and the
    48-key items of the key-split kernel that launches with few items take."""
    monkeypatch.setattr(hip, "DKDV256_MIN_ITEMS", 0 if request.param == "kv64" else 1 << 30)


def close(got, want, what, bar=2e-2):
    got = got.detach().float().cpu()
    want = want.detach().float().cpu()
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = (got - want).abs().max().item() if got.numel() else 0.0
    scale = max(1.0, want.abs().max().item() if want.numel() else 0.0)
    print(f"    {what}: max-abs {err:.4g} (bar {bar * scale:.4g} = {bar} x max(1, max|ref| {scale:.3g}))", flush=True)
    assert err <= bar * scale, f"{what}: max-abs {err:.4g} > {bar} x {scale:.3g}"
    return err


def chain(d, t, chunks, hq, hkv, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(t, hq, d, generator=g).to(dtype)
    ks = [torch.randn(n, hkv, d, generator=g).to(dtype) for n in chunks]
    vs = [torch.randn(n, hkv, d, generator=g).to(dtype) for n in chunks]
    dout = torch.randn(t, hq, d, generator=g).to(dtype)
    return q, ks, vs, dout


def run_chain(cuda, d, t, chunks, hq, hkv, seed, dtype=torch.bfloat16):
    q, ks, vs, dout = chain(d, t, chunks, hq, hkv, seed, dtype)
    scale = d ** -0.5
    want, wq, wks, wvs = ref.attention_with_grads(q, ks, vs, dout, scale)
    qc = q.to(cuda).requires_grad_()
    kc = [k.to(cuda).requires_grad_() for k in ks]
    vc = [v.to(cuda).requires_grad_() for v in vs]
    out, _ = hip.attention(qc, hip.chain_layout(t, chunks, hq, hkv), kc, vc, scale)
    assert out.shape == (t, hq, d) and out.dtype == dtype
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out, want, "out")
    close(qc.grad, wq, "dq")
    for i in range(len(chunks)):
        close(kc[i].grad, wks[i], f"dk[{i}]")
        close(vc[i].grad, wvs[i], f"dv[{i}]")


CHAINS = [
    # head dim, query rows, chunk lengths, hq, hkv
    (256, 150, [300, 150], 24, 4),   # the reference's FA4 test heads (group 6)
    (256, 64, [64], 8, 2),           # group 4: 48-key dK/dV items
    (256, 33, [80, 33], 4, 4),       # group 1
    (192, 100, [50, 100], 16, 2),    # group 8
    (96, 70, [33, 70], 6, 2),        # group 3
    (64, 130, [7, 64, 130], 32, 8),  # group 4
    (64, 1, [9], 4, 2),
    (32, 200, [300, 17, 200], 40, 8),  # group 5
    (32, 96, [96], 4, 2),            # the tiny test models' shape (4/2 heads, d32)
]


@pytest.mark.parametrize("d,t,chunks,hq,hkv", CHAINS)
def test_chain_head_dims(cuda, d, t, chunks, hq, hkv):
    print(f"attention chain d={d} t={t} chunks={chunks} hq={hq} hkv={hkv}", flush=True)
    run_chain(cuda, d, t, chunks, hq, hkv, seed=d + t + hq)


def test_fp16_head_dim_64(cuda):
    print("attention chain fp16 d=64 t=77 chunks=[120, 77] hq=8 hkv=2", flush=True)
    run_chain(cuda, 64, 77, [120, 77], 8, 2, seed=5, dtype=torch.float16)


def test_fp16_head_dim_256(cuda):
    """fp16 at head dim 256 with GQA group 6: the 32-keys-per-wave dK/dV
    kernel's fp16 products, over runs that end inside a wave's key blocks."""
    print("attention chain fp16 d=256 t=90 chunks=[130, 90] hq=12 hkv=2", flush=True)
    run_chain(cuda, 256, 90, [130, 90], 12, 2, seed=6, dtype=torch.float16)


def test_fused_projection_views_head_dim_256(cuda):
    """Q, K and V at head dim 256 (GQA group 6) as column slices of one fused
    projection output [rows, (Hq + 2 Hkv) D]: read in place through their
    strides; gradients land in the slices of the fused gradient."""
    t, s_len, hq, hkv, d = 150, 400, 12, 2, 256
    print(f"fused projection views d={d} t={t} keys={s_len} hq={hq} hkv={hkv}", flush=True)
    g = torch.Generator().manual_seed(23)
    width = (hq + 2 * hkv) * d
    qkv_q = torch.randn(t, width, generator=g).to(torch.bfloat16)
    qkv_k = torch.randn(s_len, width, generator=g).to(torch.bfloat16)
    dout = torch.randn(t, hq, d, generator=g).to(torch.bfloat16)
    scale = d ** -0.5
    split = lambda x: (x[:, : hq * d].view(-1, hq, d), x[:, hq * d : (hq + hkv) * d].view(-1, hkv, d),
                       x[:, (hq + hkv) * d :].view(-1, hkv, d))
    q_ref, _, _ = split(qkv_q)
    _, k_ref, v_ref = split(qkv_k)
    want, wq, wks, wvs = ref.attention_with_grads(q_ref, [k_ref], [v_ref], dout, scale)
    a = qkv_q.to(cuda).requires_grad_()
    b = qkv_k.to(cuda).requires_grad_()
    q, _, _ = split(a)
    _, k, v = split(b)
    out, _ = hip.attention(q, hip.chain_layout(t, [s_len], hq, hkv), [k], [v], scale)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out, want, "out")
    gq, _, _ = split(a.grad)
    _, gk, gv = split(b.grad)
    close(gq, wq, "dq")
    close(gk, wks[0], "dk")
    close(gv, wvs[0], "dv")
    assert a.grad[:, hq * d :].abs().max().item() == 0.0
    assert b.grad[:, : hq * d].abs().max().item() == 0.0


def test_fa4_branch_shape_reduced(cuda):
    """The reference's bottom-right branch (tests/test_fa4_bottom_right.py:13-28:
    a query tail over prefix + tail keys, 24/4 heads, D 256) at a reduced size:
    the HIP call through the callable-backend form against the fp32 oracle."""
    prefix, tail, hq, hkv, d = 300, 200, 24, 4, 256
    print(f"fa4 branch shape: prefix {prefix} tail {tail} {hq}/{hkv} heads d{d}", flush=True)
    g = torch.Generator().manual_seed(17)
    q = torch.randn(1, hq, tail, d, generator=g).to(torch.bfloat16)
    k = torch.randn(prefix + tail, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(prefix + tail, hkv, d, generator=g).to(torch.bfloat16)
    dout = torch.randn(1, hq, tail, d, generator=g).to(torch.bfloat16)
    scale = d ** -0.5
    want, wq, (wk,), (wv,) = ref.attention_with_grads(q[0].transpose(0, 1), [k], [v], dout[0].transpose(0, 1), scale)
    qc, kc, vc = (t.to(cuda).requires_grad_() for t in (q, k, v))
    out = hip.causal_attention(qc, [kc], [vc], scale)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out[0].transpose(0, 1), want, "out")
    close(qc.grad[0].transpose(0, 1), wq, "dq")
    close(kc.grad, wk, "dk")
    close(vc.grad, wv, "dv")


@pytest.mark.parametrize("d,hq,hkv", [(256, 24, 4), (80, 8, 2)])
def test_forest_head_dims(cuda, d, hq, hkv):
    """A two-level forest (shared prompt, four completions, two sharing a first
    turn) at D 256 with 24/4 heads, and at D 80 (run zero-padded at 96) with
    8/2 heads, against the dense-mask oracle."""
    spec = []
    import random

    rng = random.Random(3)
    prompt = [rng.randrange(50000) for _ in range(120)]
    shared = [rng.randrange(50000) for _ in range(30)]
    for i in range(4):
        segs = [("prompt", prompt, False)]
        if i < 2:
            segs.append(("action", shared, True))
        segs.append(("action", [50000 + i] + [rng.randrange(50000) for _ in range(rng.randint(20, 90))], True))
        spec.append((0, i, segs))
    kinds = {"prompt": prod.SegmentKind.PROMPT, "action": prod.SegmentKind.ACTION}
    plan = prod.compile_plan(prod.build_forest(
        [prod.Trajectory([prod.Segment(tuple(t), kinds[k], s) for k, t, s in segs], group_id=g, traj_id=i)
         for g, i, segs in spec]))
    oplan = ofo.compile_plan(ofo.build_forest(
        [ofo.Trajectory([ofo.Segment(tuple(t), k, s) for k, t, s in segs], g, i) for g, i, segs in spec]))
    p = plan.n_physical
    print(f"forest d{d}: {p} tokens, {plan.n_nodes} nodes, {hq}/{hkv} heads", flush=True)
    mask = torch.tensor(ofo.visibility_mask(oplan))
    g = torch.Generator().manual_seed(9)
    q = torch.randn(p, hq, d, generator=g).to(torch.bfloat16)
    k = torch.randn(p, hkv, d, generator=g).to(torch.bfloat16)
    v = torch.randn(p, hkv, d, generator=g).to(torch.bfloat16)
    dout = torch.randn(p, hq, d, generator=g).to(torch.bfloat16)
    scale = d ** -0.5
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


PADDED = [
    # head dim (runs at the next kernel width), query rows, chunk lengths, hq, hkv, dtype
    (80, 70, [33, 70], 8, 2, torch.bfloat16),     # -> 96
    (100, 50, [60, 50], 4, 1, torch.float16),     # -> 128, rows of 100 elements (not 16-byte multiples)
    (112, 64, [64], 8, 2, torch.bfloat16),        # -> 128, the one-wave-per-head kernels
    (160, 40, [90, 40], 8, 8, torch.bfloat16),    # -> 192
    (8, 17, [20, 17], 4, 2, torch.bfloat16),      # -> 32
    (200, 33, [33], 4, 2, torch.bfloat16),        # -> 256
]


@pytest.mark.parametrize("d,t,chunks,hq,hkv,dtype", PADDED)
def test_other_head_dims_run_zero_padded(cuda, d, t, chunks, hq, hkv, dtype):
    """Head dims the kernels are not built for run at the next kernel width
    over zero-padded Q, K and V; output and gradients against the oracle at
    the true head dim (scale d^-1/2 of the true head dim)."""
    print(f"attention chain d={d} (padded to {hip.kernel_head_dim(d)}) t={t} chunks={chunks} hq={hq} hkv={hkv} "
          f"{dtype}", flush=True)
    run_chain(cuda, d, t, chunks, hq, hkv, seed=d + t, dtype=dtype)


def test_head_dims_above_256_refused(cuda):
    q = torch.randn(8, 4, 264, device=cuda, dtype=torch.bfloat16)
    k = torch.randn(8, 1, 264, device=cuda, dtype=torch.bfloat16)
    assert hip.kernel_head_dim(264) is None and hip.kernel_head_dim(0) is None
    with pytest.raises(ValueError, match="head dims"):
        hip.attention(q, hip.chain_layout(8, [8], 4, 1), [k], [k], 0.1)
