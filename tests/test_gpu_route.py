"""GPU parity of the router (top-k softmax) and the stable expert permutation.

Routing ids and the permutation are integer results: bit-exact against the
oracle.  Weights are fp32 softmax probabilities: within 2e-6 relative of the
oracle's fp64 softmax rounded to fp32.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bits_u16
from llada_quant_amd.runtime.routing import expert_token_stats, gather_topk_weights, moe_permute, route_topk
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def zipf_logits(T: int, E: int, seed: int, s: float = 1.1) -> torch.Tensor:
    """Router logits ~N(0,1) plus a per-expert bias making popularity Zipf(s)."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(E, generator=g)
    p = torch.arange(1, E + 1, dtype=torch.float64) ** (-s)
    p = p / p.sum()
    bias = torch.log(p)[perm].float()
    return torch.randn(T, E, generator=g) + bias


@pytest.mark.parametrize("T,E,k,renorm", [(256, 16, 2, True), (512, 64, 8, False), (4096, 64, 8, True),
                                          (64, 64, 8, False), (33, 128, 6, True), (17, 256, 8, False),
                                          (5, 8, 8, True), (1, 64, 1, False)])
def test_route_topk_matches_oracle(dev, T, E, k, renorm):
    g = torch.Generator().manual_seed(T * 7 + E)
    logits = torch.randn(T, E, generator=g)
    ids, w = route_topk(logits.to(dev), k, renorm)
    ids_ref, w_ref = O.route_topk(logits.numpy(), k, renorm)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-9)


def test_route_topk_ids_equal_torch_softmax_topk(dev):
    """The router recomputes TritonFusedMoEBlock's routing: softmax(fp32).topk(k).indices."""
    logits = zipf_logits(4096, 64, seed=3)
    ids, w = route_topk(logits.to(dev), 8)
    probs = torch.softmax(logits, dim=-1, dtype=torch.float32)
    ref = probs.topk(8, dim=-1)
    assert torch.equal(ids.cpu().long(), ref.indices)
    torch.testing.assert_close(w.cpu(), ref.values, rtol=2e-6, atol=1e-9)


def test_route_topk_bf16_logits(dev):
    logits = (torch.randn(300, 64) * 2).to(torch.bfloat16)
    ids, _ = route_topk(logits.to(dev), 8)
    ids_ref, _ = O.route_topk(bits_u16(logits), 8, False, logits_dtype=O.BF16)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)


def test_route_topk_ties_go_to_the_lower_expert(dev):
    logits = torch.zeros(3, 64)
    logits[1, 10] = logits[1, 20] = 1.0
    ids, w = route_topk(logits.to(dev), 4)
    assert ids[0].tolist() == [0, 1, 2, 3]
    assert ids[1].tolist()[:2] == [10, 20] and ids[1].tolist()[2:] == [0, 1]
    ids_ref, _ = O.route_topk(logits.numpy(), 4, False)
    assert np.array_equal(ids.cpu().numpy(), ids_ref)


@pytest.mark.parametrize("T,E,k", [(64, 64, 8), (512, 64, 8), (4096, 64, 8), (32768, 64, 8), (256, 16, 2),
                                   (3, 256, 8), (1000, 7, 3)])
def test_permute_matches_oracle(dev, T, E, k):
    logits = zipf_logits(T, E, seed=T + E)
    ids, _ = route_topk(logits.to(dev), k)
    counts, offsets, sorted_ = moe_permute(ids, E)
    c_ref, o_ref, s_ref = O.moe_permute(ids.cpu().numpy(), E)
    assert np.array_equal(counts.cpu().numpy(), c_ref)
    assert np.array_equal(offsets.cpu().numpy(), o_ref)
    assert np.array_equal(sorted_.cpu().numpy(), s_ref)
    # the same order torch's stable argsort gives
    flat = ids.cpu().reshape(-1).long()
    assert torch.equal(sorted_.cpu().long(), torch.argsort(flat, stable=True))


def test_permute_is_deterministic(dev):
    ids, _ = route_topk(zipf_logits(32768, 64, seed=9).to(dev), 8)
    a = moe_permute(ids, 64)
    b = moe_permute(ids, 64)
    assert all(torch.equal(x, y) for x, y in zip(a, b))


def test_expert_token_stats_known_answer(dev):
    """analysis/moe_regime.py KAT: [[0,1],[0,2],[0,1]] over 4 experts -> [3, 2, 1, 0]."""
    stats = expert_token_stats(torch.tensor([[0, 1], [0, 2], [0, 1]], device=dev), num_experts=4)
    assert stats.counts == [3, 2, 1, 0]
    assert stats.active_experts == 3
    assert stats.mean == pytest.approx(1.5)
    assert stats.imbalance == pytest.approx(2.0)
    assert stats.to_dict()["max"] == 3


def test_gather_topk_weights(dev):
    logits = torch.randn(100, 64)
    probs = torch.softmax(logits, -1)
    topk = probs.topk(8, dim=-1)
    ids, w = gather_topk_weights(probs.to(dev), topk.indices.to(dev), renormalize=False)
    assert torch.equal(ids.cpu().long(), topk.indices)
    assert torch.equal(w.cpu(), topk.values)
    _, wn = gather_topk_weights(probs.to(dev), topk.indices.to(dev), renormalize=True)
    torch.testing.assert_close(wn.cpu(), topk.values / topk.values.sum(-1, keepdim=True), rtol=1e-6, atol=1e-7)
