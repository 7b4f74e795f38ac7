"""Tier-A token-identity gate for a quantized-kernel model.

The reference's acceptance rule for a low-bit kernel (README.md:693-706):
decode with the reference path's model and with the kernel's model, each
free-running through the same commit rule, and require that the tokens both
committed agree everywhere (``final_token_agreement == 1.0``).  The loop
follows ``capture_free_running`` (trajectory/capture.py:244-314) and the
summary follows ``replay_free_running`` (trajectory/replay.py:130-182):

- each model is driven by the caller's ``logits_fn`` and ``advance_fn``, so a
  divergence can only come from the logits;
- a step records the positions it committed and their tokens;
- ``final_token_agreement`` is 1 - (disagreeing positions) / (positions both
  committed), 1.0 when none were; ``first_divergence_step`` is the first step
  (1-based) after which the tokens committed so far disagree, -1 if never;
- ``commit_order_agreement`` is the share of steps whose committed position
  sets are equal (trajectory/metrics.py:110-126).

No decoder rule is supplied here, as in the reference: ``advance_fn(state,
logits)`` returns the next state, or None to stop.  A state carries
``input_ids`` ([1, L] or [L]) and ``mask_positions`` (same shape, bool).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Tuple

import torch

LogitsFn = Callable[[Any, Any], torch.Tensor]
AdvanceFn = Callable[[Any, torch.Tensor], Optional[Any]]


@dataclass
class Commit:
    """Positions one step committed (flat indices) and the tokens written there."""

    positions: List[int]
    tokens: List[int]


@dataclass
class GateReport:
    """Outcome of :func:`token_identity_gate` (the keys of the reference's Mode-B summary)."""

    steps: int
    final_token_agreement: float
    first_divergence_step: int
    commit_order_agreement: float
    positions_committed_by_both: int
    reference_commits: List[Commit] = field(default_factory=list)
    kernel_commits: List[Commit] = field(default_factory=list)

    @property
    def passed(self) -> bool:
        return self.final_token_agreement == 1.0

    def summary(self) -> Dict[str, float]:
        return {
            "steps": self.steps,
            "first_divergence_step": float(self.first_divergence_step),
            "final_token_agreement": self.final_token_agreement,
            "commit_order_agreement": self.commit_order_agreement,
            "positions_committed_by_both": float(self.positions_committed_by_both),
        }


def _masked(state) -> torch.Tensor:
    return state.mask_positions.reshape(-1).to(torch.bool)


def free_run(model: Any, state: Any, logits_fn: LogitsFn, advance_fn: AdvanceFn, max_steps: int) -> List[Commit]:
    """Decode one model until nothing is masked, the rule stops, or ``max_steps``."""
    commits: List[Commit] = []
    for _ in range(max_steps):
        before = _masked(state).cpu()
        if not bool(before.any()):
            break
        with torch.no_grad():
            logits = logits_fn(model, state)
            nxt = advance_fn(state, logits)
        if nxt is None:
            commits.append(Commit([], []))
            break
        after = _masked(nxt).cpu()
        newly = (before & ~after).nonzero(as_tuple=True)[0]
        ids = nxt.input_ids.reshape(-1).cpu()
        commits.append(Commit(newly.tolist(), ids[newly].tolist()))
        state = nxt
    return commits


def _compare(ref: List[Commit], ker: List[Commit]) -> Tuple[float, int, int]:
    ref_tok: Dict[int, int] = {}
    ker_tok: Dict[int, int] = {}
    first = -1
    for i in range(max(len(ref), len(ker))):
        if i < len(ref):
            ref_tok.update(zip(ref[i].positions, ref[i].tokens))
        if i < len(ker):
            ker_tok.update(zip(ker[i].positions, ker[i].tokens))
        if first < 0 and any(ref_tok[p] != ker_tok[p] for p in ref_tok.keys() & ker_tok.keys()):
            first = i + 1
    both = ref_tok.keys() & ker_tok.keys()
    wrong = sum(1 for p in both if ref_tok[p] != ker_tok[p])
    agreement = 1.0 - wrong / len(both) if both else 1.0
    return agreement, first, len(both)


def commit_order_agreement(ref: List[Commit], ker: List[Commit]) -> float:
    if not ref:
        return 1.0
    n = min(len(ref), len(ker))
    if n == 0:
        return 0.0
    same = sum(1 for i in range(n) if set(ref[i].positions) == set(ker[i].positions))
    return same / max(len(ref), len(ker))


def token_identity_gate(
    reference: Any,
    kernel: Any,
    initial_state: Any,
    logits_fn: LogitsFn,
    advance_fn: AdvanceFn,
    *,
    max_steps: int = 64,
) -> GateReport:
    """Free-run both models from ``initial_state`` and compare what they committed."""
    if max_steps < 1:
        raise ValueError(f"max_steps must be >= 1, got {max_steps}")
    ref = free_run(reference, initial_state, logits_fn, advance_fn, max_steps)
    ker = free_run(kernel, initial_state, logits_fn, advance_fn, max_steps)
    agreement, first, both = _compare(ref, ker)
    return GateReport(
        steps=max(len(ref), len(ker)),
        final_token_agreement=agreement,
        first_divergence_step=first,
        commit_order_agreement=commit_order_agreement(ref, ker),
        positions_committed_by_both=both,
        reference_commits=ref,
        kernel_commits=ker,
    )
