"""fp16 operands through the attention, fused logprob and LoRA kernels.

The kernels take bf16 or fp16 (the reference's FA4 gate accepts both,
engine/streaming.py:536-540); the same instruction sequences run with the
fp16 MFMA forms and fp16 roundings of P, dS, dlogits and the outputs.  Bars
are the bf16 tests' own (the oracle computes in fp32 from the same fp16
values, and fp16 rounds three bits finer than bf16): attention 2e-2 max-abs
(scaled by max|ref| above 1), logprob and entropy 1e-3, gradients 1e-2 of
max|ref|.  Mixed element types in one call are refused.
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as ref_attn
from oracle import logprob as ref_lp
from oracle import lora as ref_lora
from thundersync_amd import attention as hip
from thundersync_amd import fused_logprob, fused_lora

pytestmark = pytest.mark.gpu

D = 128


def close(got, want, what, bar, scale_mode="relative"):
    """max-abs within bar x scale: "absolute" (scale 1), "above_one" (max(1,
    max|ref|), the attention tests' drift metric) or "relative" (max|ref|)."""
    got, want = got.detach().double().cpu(), want.detach().double().cpu()
    assert got.shape == want.shape, (what, got.shape, want.shape)
    err = (got - want).abs().max().item() if got.numel() else 0.0
    top = want.abs().max().item() if want.numel() else 0.0
    scale = {"absolute": 1.0, "above_one": max(1.0, top), "relative": max(top, 1e-6)}[scale_mode]
    print(f"    {what}: max-abs {err:.4g} (bar {bar * scale:.4g})", flush=True)
    assert err <= bar * scale, f"{what}: max-abs {err:.4g} > {bar} x {scale:.3g}"


@pytest.mark.parametrize("t,chunks,hq,hkv", [(128, [7, 64, 130, 128], 32, 8), (37, [100, 37], 8, 2),
                                             (200, [300, 17, 200], 40, 8), (96, [96], 2, 1)])
def test_attention_chain_fp16(cuda, t, chunks, hq, hkv):
    print(f"fp16 attention chain t={t} chunks={chunks} hq={hq} hkv={hkv}", flush=True)
    g = torch.Generator().manual_seed(t + hq)
    q = torch.randn(t, hq, D, generator=g).half()
    ks = [torch.randn(n, hkv, D, generator=g).half() for n in chunks]
    vs = [torch.randn(n, hkv, D, generator=g).half() for n in chunks]
    dout = torch.randn(t, hq, D, generator=g).half()
    scale = D ** -0.5
    want, wq, wks, wvs = ref_attn.attention_with_grads(q, ks, vs, dout, scale)
    qc = q.to(cuda).requires_grad_()
    kc = [k.to(cuda).requires_grad_() for k in ks]
    vc = [v.to(cuda).requires_grad_() for v in vs]
    out, lse = hip.attention(qc, hip.chain_layout(t, chunks, hq, hkv), kc, vc, scale)
    assert out.dtype == torch.float16
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out, want, "out", 2e-2, "above_one")
    close(qc.grad, wq, "dq", 2e-2, "above_one")
    for i in range(len(chunks)):
        assert kc[i].grad.dtype == torch.float16
        close(kc[i].grad, wks[i], f"dk[{i}]", 2e-2, "above_one")
        close(vc[i].grad, wvs[i], f"dv[{i}]", 2e-2, "above_one")


def test_attention_refuses_mixed_types(cuda):
    q = torch.randn(8, 4, D, device=cuda, dtype=torch.float16)
    k = torch.randn(8, 1, D, device=cuda, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="must be torch.float16"):
        hip.attention(q, hip.chain_layout(8, [8], 4, 1), [k], [k], 0.1)
    with pytest.raises(TypeError, match="bf16 or fp16"):
        hip.attention(q.float(), hip.chain_layout(8, [8], 4, 1), [k.float()], [k.float()], 0.1)


@pytest.mark.parametrize("n,d,v", [(300, 4096, 32000), (129, 64, 501)])
def test_logprob_entropy_fp16(cuda, n, d, v):
    print(f"fp16 logprob n={n} d={d} v={v}", flush=True)
    g = torch.Generator().manual_seed(n + v)
    h = torch.randn(n, d, generator=g).half()
    w = (torch.randn(v, d, generator=g) * 0.02).half()
    t = torch.randint(0, v, (n,), generator=g)
    g_lp, g_ent = torch.randn(n, generator=g), torch.randn(n, generator=g)
    want_lp, want_ent = ref_lp.logprob_entropy_forward(h, w, t, 1024)
    want_gh, want_gw = ref_lp.logprob_entropy_backward(h, w, t, want_ent, g_lp, g_ent, 1024,
                                                       needs_weight_grad=True)
    hc, wc = h.to(cuda).requires_grad_(), w.to(cuda).requires_grad_()
    lp, ent = fused_logprob.fused_logprob_entropy(hc, wc, t.to(cuda))
    (lp * g_lp.to(cuda) + ent * g_ent.to(cuda)).sum().backward()
    torch.cuda.synchronize()
    close(lp, want_lp, "logprob", 1e-3, "absolute")
    close(ent, want_ent, "entropy", 1e-3, "absolute")
    assert hc.grad.dtype == torch.float16 and wc.grad.dtype == torch.float16
    close(hc.grad, want_gh, "grad hidden", 1e-2)
    close(wc.grad, want_gw, "grad weight", 1e-2)
    with pytest.raises(TypeError, match="one dtype"):
        fused_logprob.fused_logprob(hc.detach(), wc.detach().bfloat16(), t.to(cuda))


def test_lora_fp16(cuda):
    print("fp16 LoRA rows=500 in=512 out=256 rank=16", flush=True)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(500, 512, generator=g).half()
    w = (torch.randn(256, 512, generator=g) * 512 ** -0.5).half()
    a = torch.randn(16, 512, generator=g) * 512 ** -0.5
    b = torch.randn(256, 16, generator=g) * 0.1
    dy = torch.randn(500, 256, generator=g).half()
    xc, ac, bc = x.to(cuda).requires_grad_(), a.to(cuda).requires_grad_(), b.to(cuda).requires_grad_()
    y = fused_lora.FusedLoRALinear.apply(xc, w.to(cuda), ac, bc, 2.0)
    y.backward(dy.to(cuda))
    torch.cuda.synchronize()
    assert y.dtype == torch.float16 and xc.grad.dtype == torch.float16
    close(y, ref_lora.fused_forward(x, w), "y", 1e-2)
    want_dx, want_da, want_db = ref_lora.fused_backward(dy.float(), x.float(), w.float(), a.half().float(),
                                                        b.half().float(), 2.0)
    close(xc.grad, want_dx, "dx", 1e-2)
    close(ac.grad, want_da, "dA", 1e-2)
    close(bc.grad, want_db, "dB", 1e-2)
