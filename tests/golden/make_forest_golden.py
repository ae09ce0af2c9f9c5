"""Write tests/golden/forest_metadata.json from the reference's own builders.

Run in the build container only (the reference is not on the GPU box):

    python tests/golden/make_forest_golden.py /root/reference/src

The bit-exact conventions of the forest and plan metadata -- child order
(engine/segments.py:336), DFS pre-order (engine/plan.py:173-178), slot
order (engine/plan.py:264-319) -- are pinned only by the reference's own
outputs, so this script imports ``thundersync.engine.segments`` and
``thundersync.engine.plan`` from the given source tree, builds a fixed set
of small forests, and records their inputs and every integer field of the
compiled plan.  The fixture holds data only (token lists, flags, integer
arrays); the tests compare both the oracle restatement and the product
builder against it.
"""

from __future__ import annotations

import json
import random
import sys
from pathlib import Path

OUT = Path(__file__).resolve().parent / "forest_metadata.json"


def cases():
    """Trajectory specs: list of (group_id, traj_id, [(kind, tokens, scored), ...])."""
    rng = random.Random(1234)
    out = {}
    prompt = [5, 6, 7, 8]
    out["two_level"] = [
        (0, i, [("prompt", prompt, False), ("action", [10 + i, 11, 12], True)]) for i in range(4)
    ]
    # siblings that share part of the first action, then diverge
    out["deep_split"] = [
        (0, 0, [("prompt", prompt, False), ("action", [1, 2, 3, 4], True)]),
        (0, 1, [("prompt", prompt, False), ("action", [1, 2, 9, 9], True)]),
        (0, 2, [("prompt", prompt, False), ("action", [1, 7], True), ("observation", [3, 3], False)]),
        (0, 3, [("prompt", prompt, False), ("action", [2], True)]),
    ]
    # same tokens, different scoring flag: must not share
    out["scored_flag_splits"] = [
        (0, 0, [("prompt", prompt, False), ("action", [1, 2], True)]),
        (0, 1, [("prompt", prompt, False), ("observation", [1, 2], False)]),
    ]
    # diverging at token 0: a zero-length grouping root
    out["zero_length_root"] = [
        (0, 0, [("action", [1, 2, 3], True)]),
        (0, 1, [("action", [4, 5], True)]),
        (0, 2, [("action", [1, 2, 9], True)]),
    ]
    # a trajectory that is a prefix of another ends on an inner node
    out["prefix_trajectory"] = [
        (0, 0, [("prompt", prompt, False), ("action", [1, 2], True)]),
        (0, 1, [("prompt", prompt, False), ("action", [1, 2], True), ("observation", [3], False),
                ("action", [4, 5], True)]),
    ]
    out["duplicates"] = [
        (0, i, [("prompt", prompt, False), ("action", [1, 2, 3], True)]) for i in range(3)
    ]
    out["single"] = [(0, 0, [("prompt", [3, 4, 5], False), ("action", [6, 7], True)])]
    # groups out of id order, interleaved trajectory ids
    out["groups"] = [
        (2, 0, [("prompt", [9, 9], False), ("action", [1], True)]),
        (0, 1, [("prompt", [8], False), ("action", [2, 3], True)]),
        (2, 2, [("prompt", [9, 9], False), ("action", [4, 4], True)]),
        (1, 3, [("prompt", [7, 7, 7], False), ("action", [5], True)]),
        (0, 4, [("prompt", [8], False), ("action", [2, 6], True)]),
    ]
    # children whose first keys tie on token but not on the flag, and sort order by token
    out["sort_order"] = [
        (0, 0, [("prompt", [1], False), ("action", [30], True)]),
        (0, 1, [("prompt", [1], False), ("action", [10], True)]),
        (0, 2, [("prompt", [1], False), ("observation", [10], False)]),
        (0, 3, [("prompt", [1], False), ("action", [20], True), ("action", [1], True)]),
        (0, 4, [("prompt", [1], False), ("action", [20], True), ("action", [0], True)]),
    ]
    # random multi-turn agentic groups
    for case in range(3):
        trajs = []
        tid = 0
        for gi in range(2):
            p = [rng.randrange(50) for _ in range(rng.randrange(1, 6))]
            for _ in range(rng.randrange(2, 5)):
                segs = [("prompt", p, False)]
                for _turn in range(rng.randrange(1, 4)):
                    segs.append(("action", [rng.randrange(4) for _ in range(rng.randrange(1, 4))], True))
                    segs.append(("observation", [rng.randrange(4) for _ in range(rng.randrange(1, 3))], False))
                trajs.append((gi * 7 % 3, tid, segs))
                tid += 1
        out[f"random_{case}"] = trajs
    return out


def main(src: str) -> None:
    sys.path.insert(0, src)
    from thundersync.engine.plan import compile_plan, visibility_mask
    from thundersync.engine.segments import Segment, SegmentKind, Trajectory, build_forest

    kinds = {"prompt": SegmentKind.PROMPT, "action": SegmentKind.ACTION, "observation": SegmentKind.OBSERVATION}
    fixtures = {}
    for name, spec in cases().items():
        trajs = [
            Trajectory([Segment(tuple(toks), kinds[kind], scored) for kind, toks, scored in segs],
                       group_id=g, traj_id=t)
            for g, t, segs in spec
        ]
        forest = build_forest(trajs)
        plan = compile_plan(forest)
        mask = visibility_mask(plan)
        fixtures[name] = {
            "trajectories": [[g, t, [[k, list(toks), s] for k, toks, s in segs]] for g, t, segs in spec],
            "forest": {
                "nodes": [
                    {"tokens": n.tokens, "scored": n.scored, "parent": n.parent, "depth": n.depth,
                     "trajectories": n.trajectories, "children": n.children, "group_id": n.group_id}
                    for n in forest.nodes
                ],
                "roots": forest.roots,
                "leaf_of": {str(k): v for k, v in forest.leaf_of.items()},
            },
            "plan": {
                **{f: getattr(plan, f).tolist() for f in (
                    "token_ids", "position_ids", "node_of", "node_start", "node_end", "node_parent",
                    "node_depth", "subtree_end", "score_src", "score_tgt", "score_pos",
                    "logical_to_slot", "logical_traj")},
                "key_ranges": [[list(r) for r in kr] for kr in plan.key_ranges],
            },
            "visibility_mask_rows": ["".join("1" if b else "0" for b in row) for row in mask.tolist()],
        }
    OUT.write_text(json.dumps(fixtures, indent=1, sort_keys=True))
    print(f"wrote {OUT} ({len(fixtures)} forests)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
