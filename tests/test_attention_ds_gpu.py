"""The attention backward's two routes against the CPU oracle.

At head dims 128 and 256 the backward takes the dS route by default: the
dK/dV kernel stores dS and the dQ kernel forms dQ = dS K from it.
``THUNDERSYNC_ATTN_DS=off`` (or a problem whose single KV head's workspace
exceeds ``attention.DS_MAX_BYTES``) selects the route whose dQ kernel
recomputes S and dP; a problem whose whole workspace exceeds the cap runs the
dS route over groups of KV heads.  Both are checked against the fp32 oracle at the attention tests' bar
(2e-2 max-abs, scaled by max|ref| above 1) over GQA groups of 4, 5, 2, 1 and 6,
ragged lengths (query rows not a multiple of 32, runs not a multiple of 16,
runs before, across and after the diagonal), fp16 and a forest; dK/dV are
the same kernels' sums on both routes and must agree bit for bit.
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle import attention as ref
from oracle import forest as ofo
from thundersync_amd import _lib
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
    print(f"    {what}: max-abs {err:.4g} (bar {bar * scale:.4g})", flush=True)
    assert err <= bar * scale, f"{what}: max-abs {err:.4g} > {bar} x {scale:.3g}"


def run_both(monkeypatch, cuda, q, ks, vs, dout, layout, scale):
    """out, dq, dks, dvs of the dS route, then of the recompute route."""
    results = []
    for route in ("auto", "off"):
        monkeypatch.setenv(hip.DS_ENV, route)
        qc = q.to(cuda).requires_grad_()
        kc = [k.to(cuda).requires_grad_() for k in ks]
        vc = [v.to(cuda).requires_grad_() for v in vs]
        if route == "auto":
            lib = _lib.require_library()
            expect = bool(lib.ts_attn_ds_route(q.shape[2], layout.hq // layout.hkv))
            assert (hip._ds_route(layout, qc, lib) is not None) == expect
        out, _ = hip.attention(qc, layout, kc, vc, scale)
        out.backward(dout.to(cuda))
        torch.cuda.synchronize()
        results.append((out.detach(), qc.grad, [k.grad for k in kc], [v.grad for v in vc]))
    return results


CHAINS = [
    # head dim, query rows, chunk lengths, hq, hkv
    (128, 130, [7, 64, 130], 32, 8),     # group 4: one-wave-per-head dK/dV storing dS
    (128, 200, [300, 17, 200], 40, 8),   # group 5: key-split dK/dV, dQ 1 head x 4 row blocks
    (128, 77, [120, 77], 16, 8),         # group 2
    (128, 33, [80, 33], 4, 4),           # group 1
    (128, 1, [9], 4, 1),                 # one row
    (128, 64, [300, 17, 64], 8, 2),      # group 4, a run past row 0's keys
    (128, 40, [100, 23, 45], 6, 2),
    (256, 150, [300, 150], 24, 4),       # the reference's FA4 test heads
    (256, 64, [64], 8, 2),
    (256, 45, [33, 61], 6, 6),
    (256, 40, [100, 23, 45], 6, 2),      # runs shorter than the rows, a run past row 0's keys
    (256, 1, [9], 4, 1),                 # one row
    (256, 200, [300, 17, 200], 40, 8),   # group 5
]


@pytest.mark.parametrize("d,t,chunks,hq,hkv", CHAINS)
def test_routes_agree_with_the_oracle(monkeypatch, cuda, d, t, chunks, hq, hkv):
    print(f"routes d={d} t={t} chunks={chunks} hq={hq} hkv={hkv}", flush=True)
    g = torch.Generator().manual_seed(d + t + hq)
    q = torch.randn(t, hq, d, generator=g).bfloat16()
    ks = [torch.randn(n, hkv, d, generator=g).bfloat16() for n in chunks]
    vs = [torch.randn(n, hkv, d, generator=g).bfloat16() for n in chunks]
    dout = torch.randn(t, hq, d, generator=g).bfloat16()
    scale = d ** -0.5
    want, wq, wks, wvs = ref.attention_with_grads(q, ks, vs, dout, scale)
    (o1, dq1, dk1, dv1), (o2, dq2, dk2, dv2) = run_both(monkeypatch, cuda, q, ks, vs, dout,
                                                        hip.chain_layout(t, chunks, hq, hkv), scale)
    assert torch.equal(o1, o2)
    for route, dq in (("dS", dq1), ("recompute", dq2)):
        close(dq, wq, f"dq ({route} route)")
    for i in range(len(chunks)):
        assert torch.equal(dk1[i], dk2[i]) and torch.equal(dv1[i], dv2[i]), f"dK/dV of chunk {i} differ by route"
        close(dk1[i], wks[i], f"dk[{i}]")
        close(dv1[i], wvs[i], f"dv[{i}]")


def _random_chain(seed):
    import random

    rng = random.Random(seed)
    d = rng.choice((128, 256))
    hkv = rng.choice((1, 2))
    hq = hkv * rng.choice((1, 2, 3, 5, 6))
    chunks = [rng.randint(1, 260) for _ in range(rng.randint(1, 3))]
    return d, rng.randint(1, chunks[-1]), chunks, hq, hkv


@pytest.mark.parametrize("seed", range(8))
def test_random_chains_both_routes(monkeypatch, cuda, seed):
    """Seeded random chains (head dims 128 and 256, GQA groups 1, 2, 3, 5 and
    6, one to three chunks of 1 to 260 keys, any query count up to the last
    chunk): both routes against the oracle, dK/dV identical across routes."""
    test_routes_agree_with_the_oracle(monkeypatch, cuda, *_random_chain(seed))


def test_fp16_route(monkeypatch, cuda):
    print("routes fp16 d=256 t=96 chunks=[50, 96] hq=6 hkv=2", flush=True)
    g = torch.Generator().manual_seed(4)
    q = torch.randn(96, 6, 256, generator=g).half()
    ks = [torch.randn(n, 2, 256, generator=g).half() for n in (50, 96)]
    vs = [torch.randn(n, 2, 256, generator=g).half() for n in (50, 96)]
    dout = torch.randn(96, 6, 256, generator=g).half()
    want, wq, wks, wvs = ref.attention_with_grads(q, ks, vs, dout, 256 ** -0.5)
    (_, dq1, dk1, dv1), (_, dq2, _, _) = run_both(monkeypatch, cuda, q, ks, vs, dout,
                                                  hip.chain_layout(96, [50, 96], 6, 2), 256 ** -0.5)
    assert dq1.dtype == torch.float16
    close(dq1, wq, "dq (dS route)")
    close(dq2, wq, "dq (recompute route)")
    for i in range(2):
        close(dk1[i], wks[i], f"dk[{i}]")
        close(dv1[i], wvs[i], f"dv[{i}]")


def test_forest_route(monkeypatch, cuda):
    """A random three-level forest (24/4 heads, d256) through the dS route
    against the dense-mask oracle."""
    rng = random.Random(21)
    prompt = [rng.randrange(50000) for _ in range(90)]
    spec = []
    for i in range(5):
        segs = [("prompt", prompt, False)]
        if i < 3:
            segs.append(("action", [7, 8, 9] * 11, True))
        segs.append(("action", [50000 + i] + [rng.randrange(50000) for _ in range(rng.randint(5, 70))], True))
        spec.append((0, i, segs))
    kinds = {"prompt": prod.SegmentKind.PROMPT, "action": prod.SegmentKind.ACTION}
    plan = prod.compile_plan(prod.build_forest(
        [prod.Trajectory([prod.Segment(tuple(t), kinds[k], s) for k, t, s in segs], group_id=g, traj_id=i)
         for g, i, segs in spec]))
    oplan = ofo.compile_plan(ofo.build_forest(
        [ofo.Trajectory([ofo.Segment(tuple(t), k, s) for k, t, s in segs], g, i) for g, i, segs in spec]))
    p, hq, hkv, d = plan.n_physical, 24, 4, 256
    print(f"forest route: {p} tokens, {plan.n_nodes} nodes", flush=True)
    mask = torch.tensor(ofo.visibility_mask(oplan))
    g = torch.Generator().manual_seed(2)
    q, k, v, dout = (torch.randn(p, h, d, generator=g).bfloat16() for h in (hq, hkv, hkv, hq))
    monkeypatch.setenv(hip.DS_ENV, "auto")
    qd, kd, vd = (t.to(cuda).requires_grad_() for t in (q, k, v))
    assert hip._ds_route(hip.forest_layout(plan, hq, hkv), qd, _lib.require_library()) is not None
    out = hip.forest_attention(qd, kd, vd, plan.to(cuda), scale=d ** -0.5)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    want = ref.masked_attention(qf, kf, vf, mask, d ** -0.5)
    want.backward(dout.float())
    close(out, want, "out")
    close(qd.grad, qf.grad, "dq")
    close(kd.grad, kf.grad, "dk")
    close(vd.grad, vf.grad, "dv")


def test_workspace_cap_selects_the_recompute_route(monkeypatch, cuda):
    lay = hip.chain_layout(64, [64], 6, 2)
    q = torch.randn(64, 6, 256, device=cuda, dtype=torch.bfloat16)
    lib = _lib.require_library()
    monkeypatch.setenv(hip.DS_ENV, "auto")
    monkeypatch.setattr(hip, "DS_FREE_FRACTION", 0.0)  # the cap alone decides
    assert hip._ds_route(lay, q, lib) is not None
    monkeypatch.setattr(hip, "DS_MAX_BYTES", 1024)  # not even one KV head's dS
    assert hip._ds_route(lay, q, lib) is None
    monkeypatch.setenv(hip.DS_ENV, "off")
    monkeypatch.setattr(hip, "DS_MAX_BYTES", 16 << 30)
    assert hip._ds_route(lay, q, lib) is None
    monkeypatch.setenv(hip.DS_ENV, "auto")
    monkeypatch.setattr(hip, "DS_MAX_BYTES", 16 << 30)
    assert hip._ds_route(lay, q[..., :128].contiguous(), lib) is not None  # head dim 128, group 3
    assert hip._ds_route(lay, q[..., :64].contiguous(), lib) is None  # head dim 64: no dS kernels


@pytest.mark.parametrize("d,t,chunks,hq,hkv", [(128, 200, [300, 17, 200], 32, 8), (256, 150, [300, 150], 24, 4)])
def test_kv_head_groups_match_one_call(monkeypatch, cuda, d, t, chunks, hq, hkv):
    """A workspace cap that holds two KV heads' dS runs the route in calls over
    two KV heads at a time; every gradient equals the one-call route's bit for
    bit (the heads are independent and each sees the same kernels)."""
    print(f"kv-head groups d={d} t={t} chunks={chunks} hq={hq} hkv={hkv}", flush=True)
    g = torch.Generator().manual_seed(31 + d)
    q = torch.randn(t, hq, d, generator=g).bfloat16()
    ks = [torch.randn(n, hkv, d, generator=g).bfloat16() for n in chunks]
    vs = [torch.randn(n, hkv, d, generator=g).bfloat16() for n in chunks]
    dout = torch.randn(t, hq, d, generator=g).bfloat16()
    layout = hip.chain_layout(t, chunks, hq, hkv)
    lib = _lib.require_library()
    monkeypatch.setenv(hip.DS_ENV, "auto")
    monkeypatch.setattr(hip, "DS_FREE_FRACTION", 0.0)  # the cap alone decides
    results = []
    for cap in (None, (2 * (hq // hkv) * layout.ds_tables(cuda)["head"] + 512) * 2):
        if cap is not None:
            monkeypatch.setattr(hip, "DS_MAX_BYTES", cap)
        qc = q.to(cuda).requires_grad_()
        kc = [k.to(cuda).requires_grad_() for k in ks]
        vc = [v.to(cuda).requires_grad_() for v in vs]
        assert hip._ds_route(layout, qc, lib)[1] == (hkv if cap is None else 2)
        out, _ = hip.attention(qc, layout, kc, vc, d ** -0.5)
        out.backward(dout.to(cuda))
        torch.cuda.synchronize()
        results.append((qc.grad, [k.grad for k in kc], [v.grad for v in vc]))
    (dq1, dk1, dv1), (dq2, dk2, dv2) = results
    assert torch.equal(dq1, dq2)
    for i in range(len(chunks)):
        assert torch.equal(dk1[i], dk2[i]) and torch.equal(dv1[i], dv2[i])
