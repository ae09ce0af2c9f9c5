"""HIP attention against the CPU oracle (bottom-right causal GQA, fp32).

Bar (the north star's): outputs and input gradients within 2e-2 max-abs
of the fp32 oracle on identical bf16 inputs.  Where a tensor's magnitude
exceeds 1 (summed key gradients of a long shared prefix), the bar scales with
max|ref| -- the bf16 rounding of the stored result alone is 2^-9 relative --
which is the reference's own drift metric (tests/test_fa4_bottom_right.py:
66-70 of the reference).  Kernels use no atomics: repeated runs are
bit-identical.
"""

from __future__ import annotations

import math

import pytest
import torch

from oracle import attention as ref
from thundersync_amd import attention as hip

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


def make(t, chunks, hq, hkv, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, t, hq, D, generator=g).to(torch.bfloat16)
    ks = [torch.randn(n, hkv, D, generator=g).to(torch.bfloat16) for n in chunks]
    vs = [torch.randn(n, hkv, D, generator=g).to(torch.bfloat16) for n in chunks]
    dout = torch.randn(1, t, hq, D, generator=g).to(torch.bfloat16)
    return q, ks, vs, dout


CHAINS = [
    (64, [64], 4, 4),
    (37, [100, 37], 8, 2),
    (128, [7, 64, 130, 128], 32, 8),
    (1, [9], 4, 2),
    (2, [5, 3], 4, 2),
    (200, [300, 17, 200], 40, 8),
    (96, [96], 2, 1),
    (513, [1024, 513], 32, 8),
    (70, [33, 70], 8, 8),
]


@pytest.mark.parametrize("t,chunks,hq,hkv", CHAINS)
def test_chain_matches_oracle(cuda, t, chunks, hq, hkv):
    print(f"attention chain t={t} chunks={chunks} hq={hq} hkv={hkv}", flush=True)
    q, ks, vs, dout = make(t, chunks, hq, hkv, seed=t + sum(chunks) + hq)
    scale = D ** -0.5
    want, wq, wks, wvs = ref.attention_with_grads(q[0], ks, vs, dout[0], scale)
    qc = q.to(cuda).requires_grad_()
    kc = [k.to(cuda).requires_grad_() for k in ks]
    vc = [v.to(cuda).requires_grad_() for v in vs]
    out = hip.causal_attention(qc.transpose(1, 2), kc, vc, scale)
    assert out.shape == (1, hq, t, D)
    out.transpose(1, 2).backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out[0].transpose(0, 1), want, "out")
    close(qc.grad[0], wq, "dq")
    for i, (k, v) in enumerate(zip(kc, vc)):
        close(k.grad, wks[i], f"dk[{i}]")
        close(v.grad, wvs[i], f"dv[{i}]")


@pytest.mark.parametrize("batch", [1, 2])
def test_head_major_query_and_adapter_layouts(cuda, batch):
    """A head-major query ([B, Hq, T, D] contiguous, as the reference's
    callable backend and FA4 adapter receive it) gets its gradient in its own
    layout, without a copy through a batch index; the HF adapter (B = 1 and
    B = 2) returns [B, T, Hq, D] and every gradient matches the oracle."""
    print(f"head-major query layouts, batch {batch}", flush=True)
    t, s, hq, hkv = 150, 150, 8, 2
    g = torch.Generator().manual_seed(11 + batch)
    q = torch.randn(batch, hq, t, D, generator=g).to(torch.bfloat16)
    k = torch.randn(batch, hkv, s, D, generator=g).to(torch.bfloat16)
    v = torch.randn(batch, hkv, s, D, generator=g).to(torch.bfloat16)
    dout = torch.randn(batch, t, hq, D, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    qc, kc, vc = (x.to(cuda).requires_grad_() for x in (q, k, v))
    out, _ = hip.hip_attention_forward(None, qc, kc, vc, None, scaling=scale)
    assert out.shape == (batch, t, hq, D)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    assert qc.grad.stride() == qc.stride() and kc.grad.shape == kc.shape
    for b in range(batch):
        want, wq, wks, wvs = ref.attention_with_grads(q[b].transpose(0, 1), [k[b].transpose(0, 1)],
                                                      [v[b].transpose(0, 1)], dout[b], scale)
        close(out[b], want, f"out[{b}]")
        close(qc.grad[b].transpose(0, 1), wq, f"dq[{b}]")
        close(kc.grad[b].transpose(0, 1), wks[0], f"dk[{b}]")
        close(vc.grad[b].transpose(0, 1), wvs[0], f"dv[{b}]")


def test_lse_and_determinism(cuda):
    t, chunks, hq, hkv = 300, [512, 300], 32, 8
    q, ks, vs, dout = make(t, chunks, hq, hkv, seed=3)
    scale = D ** -0.5
    _, want_lse = ref.chained_attention(q[0], ks, vs, scale)
    layout = hip.chain_layout(t, chunks, hq, hkv)
    runs = []
    for _ in range(2):
        qc = q[0].to(cuda).requires_grad_()
        kc = [k.to(cuda).requires_grad_() for k in ks]
        vc = [v.to(cuda).requires_grad_() for v in vs]
        out, lse = hip.attention(qc, layout, kc, vc, scale)
        out.backward(dout[0].to(cuda))
        torch.cuda.synchronize()
        runs.append((out.detach(), lse, qc.grad, [k.grad for k in kc], [v.grad for v in vc]))
    torch.testing.assert_close(runs[0][1].cpu(), want_lse, rtol=0, atol=1e-3)
    a, b = runs
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and torch.equal(a[2], b[2])
    for x, y in zip(a[3] + a[4], b[3] + b[4]):
        assert torch.equal(x, y)


def test_fused_projection_views(cuda):
    """Q, K and V as column slices of one fused projection output
    [rows, (Hq + 2 Hkv) D] (row stride (Hq + 2 Hkv) D, head stride D): the
    kernels read them in place through their strides; gradients land in the
    slices of the fused tensor's gradient."""
    t, s_len, hq, hkv = 150, 400, 32, 8
    g = torch.Generator().manual_seed(21)
    width = (hq + 2 * hkv) * D
    qkv_q = torch.randn(t, width, generator=g).to(torch.bfloat16)      # rows of the queries
    qkv_k = torch.randn(s_len, width, generator=g).to(torch.bfloat16)  # rows of the keys
    dout = torch.randn(t, hq, D, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    split = lambda x: (x[:, : hq * D].view(-1, hq, D), x[:, hq * D : (hq + hkv) * D].view(-1, hkv, D),
                       x[:, (hq + hkv) * D :].view(-1, hkv, D))
    q_ref, _, _ = split(qkv_q)
    _, k_ref, v_ref = split(qkv_k)
    want, wq, wks, wvs = ref.attention_with_grads(q_ref, [k_ref], [v_ref], dout, scale)

    a = qkv_q.to(cuda).requires_grad_()
    b = qkv_k.to(cuda).requires_grad_()
    q, _, _ = split(a)
    _, k, v = split(b)
    assert q.stride() == (width, D, 1) and k.stride() == (width, D, 1)
    out, _ = hip.attention(q, hip.chain_layout(t, [s_len], hq, hkv), [k], [v], scale)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out, want, "out")
    gq, _, _ = split(a.grad)
    _, gk, gv = split(b.grad)
    close(gq, wq, "dq")
    close(gk, wks[0], "dk")
    close(gv, wvs[0], "dv")
    # the unused slices of the fused gradients stay zero
    assert a.grad[:, hq * D :].abs().max().item() == 0.0
    assert b.grad[:, : hq * D].abs().max().item() == 0.0


@pytest.mark.parametrize("slope", [40.0, -40.0])
def test_drifting_scores(cuda, slope):
    """Scores that climb (or fall) steeply along the keys: every query row is
    one direction u plus noise and key j carries slope * j / S along u, so a
    row's maximum grows by tens of log2 units over its keys.  A rising row
    exceeds its reference point by more than the forward's slack on most
    tiles (moving it and rescaling O and the row sum mid-row); a falling row
    never does, and its late keys underflow to zero weight.  Magnitudes are
    chosen so that the bf16 rounding of dS before the dQ / dK products (as
    in flash backward kernels) stays well inside the bar: computed on the
    CPU, it alone moves dQ by 0.016 of max|dQ| 2.3 here (0.021 of 1.2 with
    keys of norm 80)."""
    t, chunks, hq, hkv = 200, [700, 200], 32, 8
    s_len = sum(chunks)
    g = torch.Generator().manual_seed(11)
    u = torch.randn(D, generator=g)
    u = u / u.norm()
    q = (8.0 * u + 0.3 * torch.randn(1, t, hq, D, generator=g)).to(torch.bfloat16)
    ramp = slope * torch.arange(s_len, dtype=torch.float32) / s_len
    k_all = torch.randn(s_len, hkv, D, generator=g) + ramp[:, None, None] * u
    v_all = torch.randn(s_len, hkv, D, generator=g)
    ks = [k.to(torch.bfloat16) for k in k_all.split(chunks)]
    vs = [v.to(torch.bfloat16) for v in v_all.split(chunks)]
    dout = torch.randn(1, t, hq, D, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    want, wq, wks, wvs = ref.attention_with_grads(q[0], ks, vs, dout[0], scale)
    _, want_lse = ref.chained_attention(q[0], ks, vs, scale)
    layout = hip.chain_layout(t, chunks, hq, hkv)
    qc = q[0].to(cuda).requires_grad_()
    kc = [k.to(cuda).requires_grad_() for k in ks]
    vc = [v.to(cuda).requires_grad_() for v in vs]
    out, lse = hip.attention(qc, layout, kc, vc, scale)
    out.backward(dout[0].to(cuda))
    torch.cuda.synchronize()
    # the rise of a row's scores along its keys, in log2 units
    print(f"slope {slope}: scores move by ~{abs(slope) * 8.0 * scale / math.log(2):.0f} log2 units", flush=True)
    torch.testing.assert_close(lse.cpu(), want_lse, rtol=0, atol=1e-3)
    close(out, want, "out")
    close(qc.grad, wq, "dq")
    for i, (k, v) in enumerate(zip(kc, vc)):
        close(k.grad, wks[i], f"dk[{i}]")
        close(v.grad, wvs[i], f"dv[{i}]")


# per segment: (own tokens, turn chunks after the shared prompt), as the
# reference's packed-split test (tests/test_packed_flash_split.py:194-200)
PACKS = [
    [(157, [157, 157]), (157, [42, 157, 68]), (42, []), (157, [157])],
    [(64, [8000]), (512, [1000, 157]), (1024, [])],
    [(2, [5]), (3, [])],
]
PROMPT = 492


@pytest.mark.parametrize("hq,hkv", [(32, 8), (40, 8)])
@pytest.mark.parametrize("pack", PACKS)
def test_packed_matches_per_segment_oracle(cuda, pack, hq, hkv):
    print(f"packed pack={pack} hq={hq}", flush=True)
    g = torch.Generator().manual_seed(sum(n for n, _ in pack))
    total = sum(n for n, _ in pack)

    def leaf(*shape):
        return torch.randn(*shape, generator=g).to(torch.bfloat16)

    query = leaf(1, total, hq, D)
    key, value = leaf(total, hkv, D), leaf(total, hkv, D)
    prompt = (leaf(PROMPT, hkv, D), leaf(PROMPT, hkv, D))
    turns = [[(leaf(n, hkv, D), leaf(n, hkv, D)) for n in chunks] for _n, chunks in pack]
    dout = leaf(1, total, hq, D)
    scale = D ** -0.5

    # device leaves (the shared prompt is ONE object passed once per segment)
    qd = query.to(cuda).requires_grad_()
    kd, vd = key.to(cuda).requires_grad_(), value.to(cuda).requires_grad_()
    pk, pv = prompt[0].to(cuda).requires_grad_(), prompt[1].to(cuda).requires_grad_()
    td = [[(a.to(cuda).requires_grad_(), b.to(cuda).requires_grad_()) for a, b in segs] for segs in turns]
    ancestors = [([pk] + [a for a, _ in segs], [pv] + [b for _, b in segs]) for segs in td]
    lengths = [n for n, _ in pack]
    layout = hip.pack_layout(lengths, ancestors, device=cuda)
    out = hip.PackedAttention.apply(qd.transpose(1, 2), kd, vd, scale, layout, *layout.inputs(ancestors))
    out.transpose(1, 2).backward(dout.to(cuda))
    torch.cuda.synchronize()
    assert out.transpose(1, 2).is_contiguous()

    # oracle: each segment on its own over prompt + turns + own
    row0 = 0
    want_pk = torch.zeros(PROMPT, hkv, D)
    want_pv = torch.zeros(PROMPT, hkv, D)
    for s, (n, _chunks) in enumerate(pack):
        ks = [prompt[0]] + [a for a, _ in turns[s]] + [key[row0 : row0 + n]]
        vs = [prompt[1]] + [b for _, b in turns[s]] + [value[row0 : row0 + n]]
        o, dq, dks, dvs = ref.attention_with_grads(query[0, row0 : row0 + n], ks, vs, dout[0, row0 : row0 + n], scale)
        close(out[0, :, row0 : row0 + n].transpose(0, 1), o, f"seg {s} out")
        close(qd.grad[0, row0 : row0 + n], dq, f"seg {s} dq")
        close(kd.grad[row0 : row0 + n], dks[-1], f"seg {s} own dk")
        close(vd.grad[row0 : row0 + n], dvs[-1], f"seg {s} own dv")
        for j, (a, b) in enumerate(td[s]):
            close(a.grad, dks[1 + j], f"seg {s} turn {j} dk")
            close(b.grad, dvs[1 + j], f"seg {s} turn {j} dv")
        want_pk += dks[0]
        want_pv += dvs[0]
        row0 += n
    close(pk.grad, want_pk, "shared prompt dk")
    close(pv.grad, want_pv, "shared prompt dv")


@pytest.mark.parametrize("need", ["all", "chunks_only", "query_only"])
def test_chunked_causal_op(cuda, need):
    """``ChunkedCausalAttention.apply(query, scale, n_chunks, keep_state, backend,
    *ks, *vs)`` -- the reference's _ChunkedCausalSDPA call (engine/streaming.py:
    1354): output and per-chunk dK/dV in input order against the oracle; inputs
    that do not require grad get None."""
    t, chunks, hq, hkv = 96, [512, 130, 96], 32, 8
    q, ks, vs, dout = make(t, chunks, hq, hkv, seed=17)
    scale = D ** -0.5
    want, wq, wks, wvs = ref.attention_with_grads(q[0], ks, vs, dout[0], scale)
    qc = q.to(cuda).requires_grad_(need != "chunks_only")
    kc = [k.to(cuda).requires_grad_(need != "query_only") for k in ks]
    vc = [v.to(cuda).requires_grad_(need != "query_only") for v in vs]
    query = qc.transpose(1, 2)  # [1, Hq, T, D] view
    out = hip.ChunkedCausalAttention.apply(query, scale, len(kc), True, "auto", *kc, *vc)
    out.transpose(1, 2).backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out[0].transpose(0, 1), want, "out")
    if need != "chunks_only":
        close(qc.grad[0], wq, "dq")
    else:
        assert qc.grad is None
    for i, (k, v) in enumerate(zip(kc, vc)):
        if need == "query_only":
            assert k.grad is None and v.grad is None
        else:
            close(k.grad, wks[i], f"dk[{i}]")
            close(v.grad, wvs[i], f"dv[{i}]")


def test_chunked_causal_op_callable_backend(cuda):
    """A callable backend is called as the reference calls it and differentiated
    by re-running it under autograd (engine/streaming.py:1094-1095, 1384-1399):
    here an fp32 softmax written with torch ops on the device, whose gradients
    must then be the oracle's to fp32 accuracy."""
    calls = []

    def fp32_backend(query, ks, vs, scale):
        calls.append(torch.is_grad_enabled())
        q = query[0].float()                                  # [Hq, T, D]
        k = torch.cat(list(ks), 0).float().transpose(0, 1)    # [Hkv, S, D]
        v = torch.cat(list(vs), 0).float().transpose(0, 1)
        rep = q.shape[0] // k.shape[0]
        k = k.repeat_interleave(rep, 0)
        v = v.repeat_interleave(rep, 0)
        s = torch.matmul(q, k.transpose(1, 2).contiguous()) * scale
        tq, sk = q.shape[1], k.shape[1]
        visible = torch.arange(sk, device=q.device)[None, :] <= (sk - tq) + torch.arange(tq, device=q.device)[:, None]
        p = torch.softmax(s.masked_fill(~visible, float("-inf")), -1)
        return torch.matmul(p, v.contiguous()).to(query.dtype).unsqueeze(0)

    t, chunks, hq, hkv = 40, [64, 40], 8, 2
    q, ks, vs, dout = make(t, chunks, hq, hkv, seed=5)
    scale = D ** -0.5
    want, wq, wks, wvs = ref.attention_with_grads(q[0], ks, vs, dout[0], scale)
    qc = q.to(cuda).requires_grad_()
    kc = [k.to(cuda).requires_grad_() for k in ks]
    vc = [v.to(cuda).requires_grad_() for v in vs]
    out = hip.ChunkedCausalAttention.apply(qc.transpose(1, 2), scale, 2, False, fp32_backend, *kc, *vc)
    out.transpose(1, 2).backward(dout.to(cuda))
    torch.cuda.synchronize()
    assert calls == [False, True]  # forward without a graph, backward re-run under autograd
    close(out[0].transpose(0, 1), want, "out")
    close(qc.grad[0], wq, "dq")
    for i, (k, v) in enumerate(zip(kc, vc)):
        close(k.grad, wks[i], f"dk[{i}]")
        close(v.grad, wvs[i], f"dv[{i}]")


def test_ragged_backward(cuda):
    """``RaggedAttention.apply(scale, n, *qs, *ks, *vs)`` -- the reference's
    _RaggedAttentionIndependentVJP (engine/streaming.py:1253-1297): outputs and
    every segment's dQ, dK, dV against the oracle run on that segment alone."""
    g = torch.Generator().manual_seed(9)
    lens = [(4, 12), (8, 16), (33, 40), (128, 700), (1, 1)]
    qs = [torch.randn(1, 32, t, D, generator=g).to(torch.bfloat16) for t, _ in lens]
    ks = [torch.randn(s, 8, D, generator=g).to(torch.bfloat16) for _, s in lens]
    vs = [torch.randn(s, 8, D, generator=g).to(torch.bfloat16) for _, s in lens]
    gs = [torch.randn(1, 32, t, D, generator=g).to(torch.bfloat16) for t, _ in lens]
    qc = [q.to(cuda).requires_grad_() for q in qs]
    kc = [k.to(cuda).requires_grad_() for k in ks]
    vc = [v.to(cuda).requires_grad_() for v in vs]
    outs = hip.RaggedAttention.apply(D ** -0.5, len(lens), *qc, *kc, *vc)
    torch.autograd.backward(outs, [x.to(cuda) for x in gs])
    torch.cuda.synchronize()
    for i in range(len(lens)):
        o, gq, gk, gv = ref.attention_with_grads(qs[i][0].transpose(0, 1), [ks[i]], [vs[i]],
                                                 gs[i][0].transpose(0, 1), D ** -0.5)
        close(outs[i][0].transpose(0, 1), o, f"seg {i} out")
        close(qc[i].grad[0].transpose(0, 1), gq, f"seg {i} dq")
        close(kc[i].grad, gk[0], f"seg {i} dk")
        close(vc[i].grad, gv[0], f"seg {i} dv")


def test_ragged_cohort(cuda):
    g = torch.Generator().manual_seed(7)
    qs = [torch.randn(1, 8, n, D, generator=g).to(torch.bfloat16) for n in (4, 8, 33)]
    ks = [torch.randn(n, 2, D, generator=g).to(torch.bfloat16) for n in (12, 16, 40)]
    vs = [torch.randn(n, 2, D, generator=g).to(torch.bfloat16) for n in (12, 16, 40)]
    outs = hip.ragged_causal_attention([q.to(cuda) for q in qs], [k.to(cuda) for k in ks],
                                       [v.to(cuda) for v in vs], D ** -0.5)
    for q, k, v, o in zip(qs, ks, vs, outs):
        want, _ = ref.bottom_right_attention(q[0].transpose(0, 1), k, v, D ** -0.5)
        close(o[0].transpose(0, 1), want, "ragged out")


def test_cpu_and_dtype_refused():
    q = torch.randn(1, 4, 8, D, dtype=torch.bfloat16)
    k = torch.randn(8, 2, D, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        hip.causal_attention(q, [k], [k], 0.1)


def test_dispatch_trial_and_path_counts(cuda, monkeypatch):
    """Under auto, the HIP attention is taken after a device trial whose record
    names the gfx950 device; every forward and backward launch is counted."""
    from thundersync_amd import _lib, capability, dispatch

    monkeypatch.setenv(_lib.HIP_ENV, "auto")
    _lib.reset()
    capability.reset_kernel_probes()
    q = torch.randn(1, 8, 40, D, device=cuda, dtype=torch.bfloat16)
    assert dispatch.hip_attention_available(q)
    assert dispatch.hip_logprob_available(torch.randn(4, 256, device=cuda, dtype=torch.bfloat16))
    records = {r["kernel"]: r for r in capability.kernel_probe_records()}
    assert records["hip_attention"]["runs"] and records["hip_logprob"]["runs"], records
    assert str(records["hip_attention"]["device"]["arch"]).startswith("gfx950")
    assert not dispatch.hip_attention_available(q.float())
    before = dispatch.attention_path_counts()
    k = torch.randn(40, 2, D, device=cuda, dtype=torch.bfloat16, requires_grad=True)
    qq = q.clone().requires_grad_()
    hip.causal_attention(qq, [k], [k], D ** -0.5).float().sum().backward()
    after = dispatch.attention_path_counts()
    assert after.get("hip", 0) == before.get("hip", 0) + 1
    assert after.get("hip_backward", 0) == before.get("hip_backward", 0) + 1
