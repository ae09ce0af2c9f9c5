"""Forest scoring of a HuggingFace decoder on the gfx950 kernels.

The forest call site of the reference's engine (engine/step.py:306-490):
the decoder stack runs once over a plan's physical token stream with the
forest attention adapter bound (:class:`~thundersync_amd.attention.
forest_context`), and the unembedding is reached only through
:func:`~thundersync_amd.fused_logprob.fused_logprob`, so no ``[P, V]``
logits tensor exists.  Public names, arguments, results and error texts
follow the reference; the code is this module's own:

* the stack and the head are found through the HF model API
  (``get_decoder`` / ``get_output_embeddings``) before the attribute
  conventions of other families (``model``, ``transformer``, ``gpt_neox``;
  ``lm_head``, ``output``, ``embed_out``);
* :func:`assert_supported` refuses, once per model, a stack whose layers do
  not all go through the attention interface (``config.layer_types`` other
  than ``full_attention``, or a module whose class names a recurrence): a
  forest is an attention mask, and a recurrence would carry its state across
  branch boundaries -- wrong results, not slow ones;
* the projection is one helper over (hidden rows, targets), called once for
  the gated form and, for the ungated form, a second time for the scored
  positions whose stream successor is not their target (the last token of
  a shared node, engine/step.py:437-456).

The model must run its attention through the registered adapter
(``register_attention()``, then
``model.set_attn_implementation(HIP_FOREST_ATTENTION_NAME)``); the adapter
refuses to run outside ``forest_context``.
"""

from __future__ import annotations

import weakref
from dataclasses import dataclass

import torch

from .attention import forest_context
from .fused_logprob import fused_logprob

# class-name fragments of modules that carry state along the sequence
# outside the attention interface (engine/step.py:203-212)
RECURRENT_MARKERS = ("deltanet", "gateddelta", "mamba", "linearattention", "linear_attention", "retention",
                     "rwkv", "ssm")

_SUPPORTED: "weakref.WeakKeyDictionary[torch.nn.Module, bool]" = weakref.WeakKeyDictionary()


def assert_supported(model: torch.nn.Module, *, recheck: bool = False) -> None:
    """Raise NotImplementedError for a model the forest path cannot score
    (engine/step.py:306-357, the batch/forest mode).  Memoised per model."""
    if not recheck and _SUPPORTED.get(model):
        return
    config = getattr(model, "config", None)
    kinds = tuple(getattr(config, "layer_types", None) or ())
    other = sorted({k for k in kinds if k != "full_attention"})
    if other:
        raise NotImplementedError(
            f"model has non-attention layer types {other}; the batch/forest path cannot fork "
            "recurrent state across branches"
        )
    for name, module in model.named_modules():
        kind = type(module).__name__.lower()
        if any(marker in kind for marker in RECURRENT_MARKERS):
            raise NotImplementedError(
                f"module {name} ({type(module).__name__}) carries recurrent state outside the "
                "attention interface; see assert_supported"
            )
    _SUPPORTED[model] = True


def base_model(model: torch.nn.Module) -> torch.nn.Module:
    """The decoder stack without the unembedding (engine/step.py:358-368)."""
    get = getattr(model, "get_decoder", None)
    if callable(get) and hasattr(model, "lm_head"):
        stack = get()
        if isinstance(stack, torch.nn.Module) and stack is not model:
            return stack
    candidates = (getattr(model, a, None) for a in ("model", "transformer", "gpt_neox"))
    return next((m for m in candidates if isinstance(m, torch.nn.Module) and not hasattr(m, "lm_head")), model)


def unembedding(model: torch.nn.Module) -> torch.Tensor:
    """The output projection's weight (engine/step.py:371-380)."""
    get = getattr(model, "get_output_embeddings", None)
    head = get() if callable(get) else None
    if head is None:
        head = next((m for m in (getattr(model, a, None) for a in ("lm_head", "output", "embed_out"))
                     if isinstance(m, torch.nn.Linear)), None)
    if head is None or not isinstance(getattr(head, "weight", None), torch.Tensor):
        raise AttributeError("could not locate the unembedding; pass `weight=` explicitly")
    return head.weight


@dataclass(frozen=True)
class StepStats:
    """Token accounting of one forest scoring pass (engine/step.py:170-200)."""

    physical_tokens: int
    logical_tokens: int
    padded_tokens: int
    projected_positions: int
    logical_scored: int

    @property
    def token_compression(self) -> float:
        """Forward tokens saved by padding removal and prefix sharing together."""
        return self.padded_tokens / max(self.physical_tokens, 1)

    @property
    def projection_reduction(self) -> float:
        """Unembedding rows saved by projecting only the scored positions."""
        return self.padded_tokens / max(self.projected_positions, 1)

    def __str__(self) -> str:
        return (f"tokens {self.padded_tokens:,} -> {self.physical_tokens:,} ({self.token_compression:.2f}x)   "
                f"projected {self.padded_tokens:,} -> {self.projected_positions:,} "
                f"({self.projection_reduction:.2f}x)")


def _project(hidden, weight, rows, targets, chunk):
    return fused_logprob(hidden if rows is None else hidden.index_select(0, rows), weight, targets, chunk=chunk)


def forest_logprobs(model: torch.nn.Module, plan, *, weight: torch.Tensor | None = None, chunk: int = 1024,
                    hidden_fn=None, return_stats: bool = False, gate: bool = True):
    """``log pi(token | context)`` of every scored token in logical order: ``[L]``,
    trajectory by trajectory, each in its own token order (engine/step.py:383-472).

    ``gate=True`` projects only the scored positions.  ``gate=False`` projects
    every physical position against the stream rolled by one and re-projects
    the scored positions whose stream successor is not their target.  With
    ``return_stats`` the result is ``(logprobs, StepStats)``.
    """
    head = weight if weight is not None else unembedding(model)
    assert_supported(model)
    if hidden_fn is None:
        stack = base_model(model)

        def hidden_fn(ids, pos):
            out = stack(input_ids=ids[None], position_ids=pos[None], attention_mask=None, use_cache=False)
            return out.last_hidden_state[0]

    with forest_context(plan):
        hidden = hidden_fn(plan.token_ids, plan.position_ids)  # [P, D]
    src, tgt = plan.score_src, plan.score_tgt
    if gate:
        lp = _project(hidden, head, src, tgt, chunk)
        projected = int(src.numel())
    else:
        lp = _project(hidden, head, None, torch.roll(plan.token_ids, -1, 0), chunk).index_select(0, src)
        successor = plan.token_ids.index_select(0, (src + 1).clamp(max=plan.n_physical - 1))
        wrong = (successor != tgt).nonzero(as_tuple=True)[0]
        if wrong.numel():
            lp = lp.index_copy(0, wrong, _project(hidden, head, src.index_select(0, wrong),
                                                  tgt.index_select(0, wrong), chunk))
        projected = plan.n_physical + int(wrong.numel())
    logical = lp.index_select(0, plan.logical_to_slot)
    if not return_stats:
        return logical
    stats = StepStats(
        physical_tokens=plan.n_physical,
        logical_tokens=plan.forest.logical_tokens,
        padded_tokens=plan.forest.padded_tokens,
        projected_positions=projected,
        logical_scored=int(plan.logical_to_slot.numel()),
    )
    return logical, stats


def split_by_trajectory(plan, logical: torch.Tensor) -> dict[int, torch.Tensor]:
    """``[L]`` logprobs as ``{trajectory id: its logprobs}`` (engine/step.py:475-490).

    The logical order keeps each trajectory's tokens together, so the pieces
    are normally the runs of equal ids in ``plan.logical_traj``.  Trajectory
    ids need not be unique (``Trajectory.traj_id`` defaults to 0): when an id
    comes back after another, its runs are concatenated in logical order, as
    the reference's mask selection does.
    """
    ids, counts = torch.unique_consecutive(plan.logical_traj, return_counts=True)
    runs = logical.split(counts.tolist())
    pieces: dict[int, list[torch.Tensor]] = {}
    for tid, run in zip((int(i) for i in ids.tolist()), runs):
        pieces.setdefault(tid, []).append(run)
    return {tid: (p[0] if len(p) == 1 else torch.cat(p)) for tid, p in sorted(pieces.items())}
