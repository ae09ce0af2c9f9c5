"""Forest scoring with a HuggingFace decoder on the gfx950 kernels.

Mirrors the forest call site of the reference's engine (engine/step.py:358-490):
the decoder runs once over the plan's physical token stream with the forest
attention adapter bound by :class:`~thundersync_amd.attention.forest_context`,
and the unembedding is reached only through :func:`fused_logprob`, gated to the
scored positions, so no ``[P, V]`` logits tensor exists.

The model must run its attention through the registered adapter
(``register_attention()`` then
``model.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)``); the adapter
refuses to run outside ``forest_context``, so a model left on another
implementation would attend across trajectories and is the caller's error, as
in the reference.
"""

from __future__ import annotations

import torch

from .attention import forest_context
from .fused_logprob import fused_logprob


def base_model(model: torch.nn.Module) -> torch.nn.Module:
    """The decoder stack without the unembedding (engine/step.py:358-368)."""
    for attr in ("model", "transformer", "gpt_neox"):
        inner = getattr(model, attr, None)
        if isinstance(inner, torch.nn.Module) and not hasattr(inner, "lm_head"):
            return inner
    return model


def unembedding(model: torch.nn.Module) -> torch.Tensor:
    """The output projection's weight (engine/step.py:371-380)."""
    for attr in ("lm_head", "output", "embed_out"):
        mod = getattr(model, attr, None)
        if isinstance(mod, torch.nn.Linear):
            return mod.weight
    if hasattr(model, "get_output_embeddings"):
        emb = model.get_output_embeddings()
        if emb is not None:
            return emb.weight
    raise AttributeError("could not locate the unembedding; pass `weight=` explicitly")


def forest_logprobs(model: torch.nn.Module, plan, *, weight: torch.Tensor | None = None, chunk: int = 1024,
                    hidden_fn=None, gate: bool = True) -> torch.Tensor:
    """``log pi(token | context)`` of every scored token, in logical order
    (engine/step.py:383-472): ``[L]``, trajectory by trajectory, each in its
    own token order.

    ``gate=True`` projects only the scored positions; ``gate=False`` projects
    every physical position against the rolled stream and re-projects the
    scored positions whose successor in the stream is not their target (the
    last token of a shared node, engine/step.py:437-456).
    """
    w = weight if weight is not None else unembedding(model)
    if hidden_fn is None:
        stack = base_model(model)

        def hidden_fn(ids, pos):
            out = stack(input_ids=ids.unsqueeze(0), position_ids=pos.unsqueeze(0), attention_mask=None,
                        use_cache=False)
            return out.last_hidden_state[0]

    with forest_context(plan):
        hidden = hidden_fn(plan.token_ids, plan.position_ids)  # [P, D]
    if gate:
        lp = fused_logprob(hidden.index_select(0, plan.score_src), w, plan.score_tgt, chunk=chunk)
    else:
        targets = torch.roll(plan.token_ids, shifts=-1, dims=0)
        lp = fused_logprob(hidden, w, targets, chunk=chunk).index_select(0, plan.score_src)
        nxt = plan.token_ids.index_select(0, (plan.score_src + 1).clamp(max=plan.n_physical - 1))
        boundary = (nxt != plan.score_tgt).nonzero(as_tuple=True)[0]
        if boundary.numel():
            fix = fused_logprob(hidden.index_select(0, plan.score_src.index_select(0, boundary)), w,
                                plan.score_tgt.index_select(0, boundary), chunk=chunk)
            lp = lp.index_copy(0, boundary, fix)
    return lp.index_select(0, plan.logical_to_slot)


def split_by_trajectory(plan, logical: torch.Tensor) -> dict[int, torch.Tensor]:
    """Regroup ``[L]`` logprobs by trajectory id (engine/step.py:475-490)."""
    out: dict[int, torch.Tensor] = {}
    traj = plan.logical_traj
    for tid in traj.unique(sorted=True).tolist():
        out[int(tid)] = logical[traj == tid]
    return out
