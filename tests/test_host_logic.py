"""Host-side helpers of the path, no GPU: the block-K alignment guards and the routing report.

Ports of tests/unit/test_moe_regime.py:89-97 (the report fields) and
:168-185 (the block-K helpers of symmetric.py:365-399, which a GEMM tuner uses
to keep a K tile inside one scale group).
"""

from __future__ import annotations

import pytest

from llada_quant_amd.algorithms.symmetric import (
    aligned_block_k_values,
    block_k_is_scale_aligned,
    validate_block_k_alignment,
)
from llada_quant_amd.runtime.routing import ExpertTokenStats, expert_token_stats


def test_block_k_must_divide_or_be_divided_by_group_size():
    for block_k in (32, 64, 128, 256):
        assert block_k_is_scale_aligned(block_k, 128)
    assert not block_k_is_scale_aligned(96, 128)
    assert not block_k_is_scale_aligned(48, 128)
    assert block_k_is_scale_aligned(96, -1), "per-tensor scaling has one scale"
    assert aligned_block_k_values(128, [32, 64, 96, 128, 256]) == [32, 64, 128, 256]
    validate_block_k_alignment(64, 128)
    with pytest.raises(ValueError, match="straddles a group boundary"):
        validate_block_k_alignment(96, 128)


def test_block_k_alignment_by_brute_force():
    """block_k is aligned to groups of g exactly when every K tile either lies inside one
    group or covers whole groups (checked tile by tile over a K both divide)."""
    for g in (16, 32, 48, 64, 96, 128):
        for bk in (8, 16, 24, 32, 48, 64, 96, 128, 192, 256):
            K = 2 * 256 * 3 * 128  # a multiple of every size here
            exact = all((t * bk) // g == (t * bk + bk - 1) // g or (t * bk % g == 0 and (t + 1) * bk % g == 0)
                        for t in range(K // bk))
            assert block_k_is_scale_aligned(bk, g) == exact, (bk, g)
    for bad in (0, -5):
        assert not block_k_is_scale_aligned(bad, 128)


def test_routing_report_fields():
    stats = ExpertTokenStats(tokens=3, top_k=2, num_experts=4, counts=[3, 2, 1, 0])
    assert stats.active_experts == 3
    assert stats.mean == pytest.approx(1.5) and stats.imbalance == pytest.approx(2.0)
    assert stats.to_dict() == {
        "tokens": 3, "top_k": 2, "num_experts": 4, "active_experts": 3, "min": 0, "p50": 2.0, "mean": 1.5,
        "p90": 3.0, "p99": 3.0, "max": 3, "imbalance_max_over_mean": 2.0,
    }
    odd = ExpertTokenStats(tokens=1, top_k=1, num_experts=3, counts=[1, 0, 0])
    assert odd.to_dict()["mean"] == 0.33 and odd.to_dict()["imbalance_max_over_mean"] == 3.0


def test_routing_report_of_nothing_routed_is_balanced():
    empty = ExpertTokenStats(tokens=0, top_k=2, num_experts=4, counts=[0, 0, 0, 0])
    assert empty.mean == 0.0 and empty.imbalance == 1.0
    none = ExpertTokenStats(tokens=0, top_k=2, num_experts=0, counts=[])
    assert none.imbalance == 1.0 and none.percentile(50) == 0.0
    assert none.to_dict()["min"] == 0 and none.to_dict()["max"] == 0


def test_routing_report_rejects_wrong_rank():
    import torch

    with pytest.raises(ValueError, match=r"\[tokens, top_k\]"):
        expert_token_stats(torch.zeros(4, dtype=torch.int32), num_experts=4)
