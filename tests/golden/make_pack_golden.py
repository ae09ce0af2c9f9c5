"""Write tests/golden/pack_layout.json from the reference's own ``_PackLayout``.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_pack_golden.py /root/reference/src

The packed attention op takes every segment's ancestor K/V chunks as autograd
inputs in one fixed order (engine/streaming.py:1636-1650): autograd sums the
gradients of a chunk several segments read (their shared prompt) in input
order, so that order is part of the op's numerical contract.  Nothing but
the reference's own code fixes it, so this script imports
``thundersync.engine.streaming`` from the given source tree, builds
``_PackLayout`` objects for a set of packs, and records:

* ``inputs``: for each input position, the (half, segment, chunk) it holds,
  where half 0 is K and half 1 is V;
* ``by_segment``: for each segment, the input positions (within one half) of
  its chunks, in the order ``by_segment`` hands them back.

The chunks handed to ``_PackLayout`` are plain string tags, so the fixture is
data only (integers); ``inputs`` and ``by_segment`` never look inside them.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "pack_layout.json"

# name -> ancestor chunk count per segment, in segment order
PACKS = {
    "single_segment": [3],
    "single_chunk_each": [1, 1, 1, 1],
    "uneven_counts": [3, 4, 1, 2],
    "increasing": [1, 2, 3, 4, 5],
    "decreasing": [5, 4, 3, 2, 1],
    "with_empty_ancestors": [2, 0, 3, 0],
    "leading_empty": [0, 1, 2],
    "many_segments": [2, 1, 3, 1, 1, 4, 2, 1, 1, 2, 3, 1],
}


def main(src: str) -> None:
    sys.path.insert(0, src)
    import torch
    from thundersync.engine.streaming import _PackLayout

    fixtures = {}
    for name, counts in PACKS.items():
        ancestors = [
            ([f"k:{s}:{c}" for c in range(n)], [f"v:{s}:{c}" for c in range(n)])
            for s, n in enumerate(counts)
        ]
        layout = _PackLayout(
            lengths=[1] * len(counts),
            prefixes=[0] * len(counts),
            counts=list(counts),
            cu_lengths=torch.zeros(len(counts) + 1, dtype=torch.int32),
            cu_prefixes=torch.zeros(len(counts) + 1, dtype=torch.int32),
            empty=torch.empty(0),
        )
        inputs = layout.inputs(ancestors)
        decoded = []
        for tag in inputs:
            half, s, c = tag.split(":")
            decoded.append([0 if half == "k" else 1, int(s), int(c)])
        total = sum(counts)
        position = {tag: i for i, tag in enumerate(inputs[:total])}
        regrouped = layout.by_segment(tuple(inputs[:total]))
        fixtures[name] = {
            "counts": list(counts),
            "inputs": decoded,
            "by_segment": [[position[tag] for tag in seg] for seg in regrouped],
        }
    OUT.write_text(json.dumps(fixtures, indent=1, sort_keys=True))
    print(f"wrote {OUT} ({len(fixtures)} packs)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
