"""Tier-A token-identity gate on the GPU (llada_quant_amd/gate.py).

A small masked-diffusion language model -- embeddings, a fixed token-mixing
step (standing in for attention, so committed tokens condition the later
steps), a quantized MoE layer with a residual, mixing again, an LM head --
decodes 32 masked positions, 4 a step, left to right, each the argmax token
of the full-sequence logits.  The
reference-path model runs each MoE layer as the reference does (dequantize to
BF16, then the fused_moe op order: oracle/torch_ref.py, on the CPU); the
kernel model runs it through
lq_moe_layer on the GPU.  Everything else is the same CPU code, so only the
MoE layers can make the decodes differ.  The gate requires
final_token_agreement == 1.0 (the reference's Tier-A rule, README.md:693-706).

The commit rule ranks nothing, so a decode can only change through an
argmax.  Two valid op orders of the layer round differently in bf16: the
torch fused order against the fp64-accumulating oracle moves this model's LM
logits by 0.028-0.042 at most (ten seeds, CPU).  The test asserts from the
reference path that every committed position's top-2 logit gap exceeds 0.08,
and at least twice the kernel's own largest logit change at the first step,
so the gate is not decided by near-ties; seeds 5 and 8 are ones whose decodes
have such margins (0.088, 0.142).

One MoE layer: its router input is identical on both paths while the tokens
agree.  With a second routed layer, an ulp of the first layer's output (the
fp32 accumulation order) can flip the second's choice where its k-th and
(k+1)-th experts are nearly tied -- a near-tie of the model (the reference's
tie_fraction), not an error of the kernel: a two-layer version of this model
(seed 1) met one, router probabilities 0.12638 and 0.12560 for the 2nd and
3rd experts, and switched a token.

The same model with a planted mistake in the reference path (gate and up
halves of W1 swapped) must fail the gate, so the MoE layers do decide tokens.
"""

from __future__ import annotations

from dataclasses import dataclass

import pytest
import torch

from llada_quant_amd.algorithms.symmetric import quantize_tensor
from llada_quant_amd.gate import token_identity_gate
from llada_quant_amd.runtime.fused_moe import moe_layer
from oracle import torch_ref

pytestmark = pytest.mark.gpu

V, PROMPT, GEN = 96, 8, 32
H, I, E, K, LAYERS, BITS, GROUP = 256, 128, 8, 2, 1, 4, 64


@dataclass
class State:
    input_ids: torch.Tensor  # [1, L]
    mask_positions: torch.Tensor  # [1, L] bool


class TinyDiffusionLM:
    def __init__(self, dev, seed: int = 0):
        g = torch.Generator().manual_seed(seed)
        L = PROMPT + GEN
        self.emb = torch.randn(V + 1, H, generator=g).to(torch.bfloat16)  # row V: the mask token
        self.pos = (0.5 * torch.randn(L, H, generator=g)).to(torch.bfloat16)
        self.mix = torch.softmax(torch.randn(L, L, generator=g), dim=-1)  # row-stochastic token mixing
        self.gate = [(0.1 * torch.randn(E, H, generator=g)).to(torch.bfloat16) for _ in range(LAYERS)]
        self.lm = (0.1 * torch.randn(V, H, generator=g)).to(torch.bfloat16)
        self.q = []
        for _ in range(LAYERS):
            # the layer's output ~0.4x the residual stream's: enough to decide tokens
            w1 = (0.05 * torch.randn(E, 2 * I, H, generator=g)).to(torch.bfloat16).to(dev)
            w2 = (0.05 * torch.randn(E, H, I, generator=g)).to(torch.bfloat16).to(dev)
            self.q.append((quantize_tensor(w1, bits=BITS, group_size=GROUP, scale_search="mse", search_grid=16),
                           quantize_tensor(w2, bits=BITS, group_size=GROUP, scale_search="mse", search_grid=16)))
        self.cpu_q = [tuple(t.cpu() for t in (q1.q, q1.scale, q2.q, q2.scale)) for q1, q2 in self.q]

    def logits(self, state: State, moe) -> torch.Tensor:
        ids = state.input_ids.reshape(-1)
        h = (self.emb[ids].float() + self.pos.float()).to(torch.bfloat16)
        for layer in range(LAYERS):
            h = (h.float() + self.mix @ h.float()).to(torch.bfloat16)
            r = h.float() @ self.gate[layer].float().T
            h = (h.float() + moe(layer, h, r).float()).to(torch.bfloat16)
        h = (h.float() + self.mix @ h.float()).to(torch.bfloat16)
        return h.float() @ self.lm.float().T


def reference_moe(model: TinyDiffusionLM, swap_gate_up: bool = False):
    def run(layer, h, r):
        q1, s1, q2, s2 = model.cpu_q[layer]
        if swap_gate_up:  # the planted mistake
            q1 = torch.cat([q1[:, I:], q1[:, :I]], dim=1)
            s1 = torch.cat([s1[:, I:], s1[:, :I]], dim=1)
        out, _ = torch_ref.packed_layer(h, r, q1, s1, q2, s2, BITS, GROUP, K)
        return out

    return run


def kernel_moe(model: TinyDiffusionLM, dev):
    def run(layer, h, r):
        q1, q2 = model.q[layer]
        out, _ = moe_layer(h.to(dev), r.to(dev), q1, q2, top_k=K)
        return out.cpu()

    return run


def start() -> State:
    ids = torch.full((1, PROMPT + GEN), V, dtype=torch.long)
    ids[0, :PROMPT] = torch.arange(3, 3 + PROMPT)
    mask = torch.zeros(1, PROMPT + GEN, dtype=torch.bool)
    mask[0, PROMPT:] = True
    return State(ids, mask)


def ordered_commit(per_step: int, gaps=None):
    """Commit the first `per_step` masked positions, each to its argmax token; record top-2 gaps."""

    def advance(state: State, logits: torch.Tensor):
        mask = state.mask_positions.reshape(-1)
        take = mask.nonzero(as_tuple=True)[0][:per_step]
        lg = logits.reshape(mask.numel(), -1)
        if gaps is not None:
            t2 = lg[take].topk(2, dim=-1).values
            gaps.append(float((t2[:, 0] - t2[:, 1]).min()))
        ids = state.input_ids.reshape(-1).clone()
        new_mask = mask.clone()
        ids[take] = lg[take].argmax(dim=-1)
        new_mask[take] = False
        return State(ids.reshape(1, -1), new_mask.reshape(1, -1))

    return advance


def model_logits(moe_and_model, state):
    model, moe = moe_and_model
    return model.logits(state, moe)


@pytest.mark.parametrize("seed", [5, 8])
def test_kernel_model_reproduces_the_reference_path_tokens(dev, seed):
    model = TinyDiffusionLM(dev, seed)
    gaps = []
    ref = token_identity_gate((model, reference_moe(model)), (model, reference_moe(model)), start(), model_logits,
                              ordered_commit(4, gaps))
    moved = float((model.logits(start(), reference_moe(model)) - model.logits(start(), kernel_moe(model, dev))).abs().max())
    assert ref.passed and min(gaps) > max(0.08, 2 * moved), (
        f"the reference decode has a near-tie: top-2 gap {min(gaps):.3g}, kernel logit change {moved:.3g}")
    rep = token_identity_gate((model, reference_moe(model)), (model, kernel_moe(model, dev)), start(),
                              model_logits, ordered_commit(4))
    assert rep.positions_committed_by_both == GEN
    assert rep.steps == GEN // 4
    assert rep.passed, rep.summary()
    assert rep.first_divergence_step == -1
    assert rep.commit_order_agreement == 1.0


def test_a_planted_mistake_in_the_reference_path_fails_the_gate(dev):
    model = TinyDiffusionLM(dev, 5)
    rep = token_identity_gate((model, reference_moe(model, swap_gate_up=True)), (model, kernel_moe(model, dev)),
                              start(), model_logits, ordered_commit(4))
    assert not rep.passed
    assert rep.first_divergence_step >= 1
