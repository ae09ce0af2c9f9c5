"""Query chunks over retained per-chunk K/V in one launch, against the CPU oracle.

Every query chunk is the reference's per-chunk call (``_ChunkedCausalSDPA``,
engine/streaming.py:1314-1423 of the reference): bottom-right causal over the
concatenation of the retained chunks on its path.  The oracle computes each
chunk on its own (fp32, explicit softmax) and sums the key/value gradients a
retained chunk receives from every query chunk that reads it.  Bar: 2e-2
max-abs, scaled by max|ref| above 1 (see test_attention_gpu.py).
"""

from __future__ import annotations

import pytest
import torch

from oracle import attention as ref
from thundersync_amd import attention as hip

from test_attention_gpu import close

pytestmark = pytest.mark.gpu

D = 128


def pack(prompts, trajectories, chunk):
    """(chunk_rows, query chunks, rows): prompts[g] tokens, then each
    trajectory of group g, all cut into `chunk`-token query chunks."""
    chunk_rows, chunks, row = [], [], 0

    def cut(n, path):
        nonlocal row
        for c0 in range(0, n, chunk):
            m = min(chunk, n - c0)
            chunk_rows.append(m)
            path.append(len(chunk_rows) - 1)
            chunks.append((row, m, tuple(path)))
            row += m

    for g, p in enumerate(prompts):
        prompt_path = []
        cut(p, prompt_path)
        for n in trajectories[g]:
            cut(n, list(prompt_path))
    return chunk_rows, chunks, row


def oracle_grads(chunks, q, ks, vs, dout, scale):
    out = torch.zeros(q.shape)
    dq = torch.zeros(q.shape)
    dks = [torch.zeros(k.shape) for k in ks]
    dvs = [torch.zeros(v.shape) for v in vs]
    for row0, m, path in chunks:
        o, gq, gk, gv = ref.attention_with_grads(q[row0 : row0 + m], [ks[c] for c in path],
                                                 [vs[c] for c in path], dout[row0 : row0 + m], scale)
        out[row0 : row0 + m] = o
        dq[row0 : row0 + m] = gq
        for c, a, b in zip(path, gk, gv):
            dks[c] += a
            dvs[c] += b
    return out, dq, dks, dvs


SMALL = [
    # prompts per group, completion lengths per group, chunk, hq, hkv
    ([96], [[100, 64, 1]], 64, 32, 8),
    ([64, 130], [[200, 17], [65]], 64, 8, 2),
    ([33], [[300]], 128, 4, 4),
]


@pytest.mark.parametrize("prompts,trajs,chunk,hq,hkv", SMALL)
def test_retained_chunks_match_oracle(cuda, prompts, trajs, chunk, hq, hkv):
    print(f"retained chunks prompts={prompts} trajs={trajs} chunk={chunk} hq={hq} hkv={hkv}", flush=True)
    chunk_rows, chunks, rows = pack(prompts, trajs, chunk)
    g = torch.Generator().manual_seed(rows + hq)
    q = torch.randn(rows, hq, D, generator=g).to(torch.bfloat16)
    ks = [torch.randn(n, hkv, D, generator=g).to(torch.bfloat16) for n in chunk_rows]
    vs = [torch.randn(n, hkv, D, generator=g).to(torch.bfloat16) for n in chunk_rows]
    dout = torch.randn(rows, hq, D, generator=g).to(torch.bfloat16)
    scale = D ** -0.5
    want, wq, wks, wvs = oracle_grads(chunks, q, ks, vs, dout, scale)
    layout = hip.retained_chunk_layout(rows, chunk_rows, chunks, hq, hkv)
    assert layout.visible_pairs() == sum(m * (sum(chunk_rows[c] for c in p) - m) + m * (m + 1) // 2
                                         for _, m, p in chunks)
    qc = q.to(cuda).requires_grad_()
    kc = [k.to(cuda).requires_grad_() for k in ks]
    vc = [v.to(cuda).requires_grad_() for v in vs]
    out = hip.retained_chunk_attention(qc, kc, vc, layout, scale)
    out.backward(dout.to(cuda))
    torch.cuda.synchronize()
    close(out, want, "out")
    close(qc.grad, wq, "dq")
    for i in range(len(chunk_rows)):
        close(kc[i].grad, wks[i], f"dk[{i}]")
        close(vc[i].grad, wvs[i], f"dv[{i}]")


def test_c4_full_size_sampled(cuda):
    """The C4 bench pack (seed 0, 140k rows, 280 retained chunks) in one launch
    per direction; sampled query chunks against the oracle: outputs and dQ of
    the longest path's last chunk and of a first completion chunk, and dK/dV
    of a trajectory's last chunk (read by that chunk alone)."""
    import bench

    print("C4 full size, seed 0", flush=True)
    lengths, chunks, layout, q, ks, vs, dout = bench.c4_inputs(0, cuda)
    scale = D ** -0.5
    out = hip.retained_chunk_attention(q, ks, vs, layout, scale)
    out.backward(dout)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and torch.isfinite(q.grad).all()
    # the longest trajectory's last chunk, and the first chunk after group 0's prompt
    longest = max(range(len(chunks)), key=lambda i: len(chunks[i][2]))
    first_completion = 2
    for i in (longest, first_completion):
        row0, m, path = chunks[i]
        print(f"  chunk {i}: {m} rows over {sum(ks[c].shape[0] for c in path)} keys", flush=True)
        o, gq, gk, gv = ref.attention_with_grads(
            q.detach()[row0 : row0 + m].cpu(), [ks[c].detach().cpu() for c in path],
            [vs[c].detach().cpu() for c in path], dout[row0 : row0 + m].cpu(), scale)
        close(out[row0 : row0 + m], o, f"out[chunk {i}]")
        close(q.grad[row0 : row0 + m], gq, f"dq[chunk {i}]")
        if i == longest:  # its own retained chunk is read by no other query chunk
            close(ks[path[-1]].grad, gk[-1], f"dk[chunk {i}]")
            close(vs[path[-1]].grad, gv[-1], f"dv[chunk {i}]")

    # group 0's first prompt chunk, KV head 0, in full: every query chunk of
    # the group reads it (the prompt's own chunks and every trajectory's)
    first = chunks[0][2][0]
    n_keys = ks[first].shape[0]
    readers = [c for c in chunks if c[2][0] == first]
    want_dk = torch.zeros(n_keys, 1, D)
    want_dv = torch.zeros(n_keys, 1, D)
    qc, dc = q.detach().cpu(), dout.cpu()
    for row0, m, path in readers:
        dk, dv = ref.prefix_key_grads(qc[row0 : row0 + m, :4], [ks[c].detach()[:, :1].cpu() for c in path],
                                      [vs[c].detach()[:, :1].cpu() for c in path], dc[row0 : row0 + m, :4],
                                      scale, n_keys)
        want_dk += dk
        want_dv += dv
    print(f"  prompt chunk {first}: {n_keys} keys read by {len(readers)} query chunks "
          f"({sum(m for _, m, _ in readers)} rows)", flush=True)
    close(ks[first].grad[:, :1], want_dk, "dk[prompt chunk, kv head 0]")
    close(vs[first].grad[:, :1], want_dv, "dv[prompt chunk, kv head 0]")
