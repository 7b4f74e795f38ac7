"""Host logic of the token-identity gate (llada_quant_amd/gate.py).

Models here are fixed logits tables, so every expected figure is counted by
hand from the commit schedule the rule produces.
"""

from __future__ import annotations

from dataclasses import dataclass

import pytest
import torch

from llada_quant_amd.gate import token_identity_gate

MASK = 99


@dataclass
class State:
    input_ids: torch.Tensor  # [1, L]
    mask_positions: torch.Tensor  # [1, L] bool


def start(L: int, prompt: int = 0) -> State:
    ids = torch.full((1, L), MASK, dtype=torch.long)
    ids[0, :prompt] = torch.arange(prompt)
    mask = torch.ones(1, L, dtype=torch.bool)
    mask[0, :prompt] = False
    return State(ids, mask)


def confident_commit(per_step: int):
    """Commit the `per_step` masked positions of highest top-1 probability (ties to the lower position)."""

    def advance(state: State, logits: torch.Tensor):
        mask = state.mask_positions.reshape(-1)
        probs = torch.softmax(logits.reshape(mask.numel(), -1).float(), dim=-1)
        conf, tok = probs.max(dim=-1)
        conf = torch.where(mask, conf, torch.full_like(conf, -1.0))
        order = torch.sort(-conf, stable=True).indices
        take = order[: min(per_step, int(mask.sum()))]
        ids = state.input_ids.reshape(-1).clone()
        new_mask = mask.clone()
        ids[take] = tok[take]
        new_mask[take] = False
        return State(ids.reshape(1, -1), new_mask.reshape(1, -1))

    return advance


def table_logits(model, state):
    return model  # a fixed [L, V] table: the same logits whatever the state


def table(L: int, V: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    t = 0.1 * torch.randn(L, V, generator=g)
    # one clear top token per row, its margin growing with the position, so the
    # confidences are distinct and the commit order is fixed by the table alone
    top = torch.randint(0, V, (L,), generator=g)
    t[torch.arange(L), top] += 2.0 + 0.5 * torch.arange(L, dtype=torch.float32)
    return t


def test_identical_models_agree_everywhere():
    t = table(12, 7, 0)
    rep = token_identity_gate(t, t.clone(), start(12), table_logits, confident_commit(3))
    assert rep.passed
    assert rep.final_token_agreement == 1.0
    assert rep.first_divergence_step == -1
    assert rep.commit_order_agreement == 1.0
    assert rep.positions_committed_by_both == 12
    assert rep.steps == 4
    # the most confident positions (the largest margins) go first; a step lists its positions ascending
    assert rep.reference_commits[0].positions == [9, 10, 11]


def test_one_flipped_token_is_counted_at_the_step_that_commits_it():
    t = table(12, 7, 1)
    k = t.clone()
    p = 4  # committed in step 3 (positions 11..9, 8..6, 5..3)
    a = int(k[p].argmax())
    b = (a + 1) % 7
    k[p, [a, b]] = k[p, [b, a]]  # the row's values permuted: another token, same confidence
    rep = token_identity_gate(t, k, start(12), table_logits, confident_commit(3))
    assert not rep.passed
    assert rep.final_token_agreement == pytest.approx(1.0 - 1.0 / 12)
    assert rep.first_divergence_step == 3
    assert rep.commit_order_agreement == 1.0


def test_same_tokens_in_another_order_lower_commit_order_only():
    t = table(8, 5, 2)
    k = t.clone()
    # make position 0 the most confident in the kernel model, same token
    k[0, k[0].argmax()] += 100.0
    rep = token_identity_gate(t, k, start(8), table_logits, confident_commit(2))
    assert rep.final_token_agreement == 1.0
    assert rep.first_divergence_step == -1
    assert rep.commit_order_agreement < 1.0


def test_prompt_positions_are_never_committed():
    t = table(10, 6, 3)
    rep = token_identity_gate(t, t, start(10, prompt=4), table_logits, confident_commit(4))
    committed = sorted(p for c in rep.reference_commits for p in c.positions)
    assert committed == list(range(4, 10))
    assert rep.positions_committed_by_both == 6


def test_rule_that_stops_and_step_limit():
    t = table(6, 4, 4)
    rep = token_identity_gate(t, t, start(6), table_logits, lambda s, lg: None)
    assert rep.steps == 1 and rep.positions_committed_by_both == 0
    assert rep.final_token_agreement == 1.0  # nothing committed by both
    rep = token_identity_gate(t, t, start(6), table_logits, confident_commit(1), max_steps=2)
    assert rep.steps == 2 and rep.positions_committed_by_both == 2
    with pytest.raises(ValueError):
        token_identity_gate(t, t, start(6), table_logits, confident_commit(1), max_steps=0)


def test_positions_committed_by_one_model_only_are_not_compared():
    t = table(6, 4, 5)
    k = t.clone()
    k[0] = -k[0]  # another token at position 0, and it is no longer confident
    # two steps of 2: the reference commits its 4 most confident, the kernel differs in the set
    rep = token_identity_gate(t, k, start(6), table_logits, confident_commit(2), max_steps=2)
    ref = {p for c in rep.reference_commits for p in c.positions}
    ker = {p for c in rep.kernel_commits for p in c.positions}
    assert rep.positions_committed_by_both == len(ref & ker)
    assert rep.summary()["positions_committed_by_both"] == float(len(ref & ker))
