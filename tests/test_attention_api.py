"""Host-side contracts of the attention operators (CPU: nothing launches)."""

from __future__ import annotations

import pytest
import torch

from thundersync_amd import attention as hip


def test_overlapping_runs_of_one_source_are_refused():
    with pytest.raises(ValueError, match="overlap"):
        hip.AttnLayout(q_rows=4, hq=4, hkv=1, source_rows=(10,),
                       runs=(hip.Run(0, 0, 6), hip.Run(0, 4, 6)),
                       seg_q=((0, 4),), seg_spans=(((0, 0), (1, 6)),))
    # adjacent runs are fine
    hip.AttnLayout(q_rows=4, hq=4, hkv=1, source_rows=(12,), runs=(hip.Run(0, 0, 6), hip.Run(0, 6, 6)),
                   seg_q=((0, 4),), seg_spans=(((0, 0), (1, 6)),))


def test_chunked_op_refuses_unknown_backend_names():
    q = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    k = torch.zeros(2, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="unknown source attention backend"):
        hip.ChunkedCausalAttention.apply(q, 0.1, 1, True, "flash", k, k)
