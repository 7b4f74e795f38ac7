"""Routing front end on the GPU: top-k softmax router, weight gather, stable permutation.

* :func:`route_topk` -- ``softmax(logits, dim=-1, dtype=float32)`` then top-k,
  the routing ``TritonFusedMoEBlock.forward`` performs and
  ``trajectory/llada.py:228-234`` restates; one wavefront per token.
* :func:`gather_topk_weights` -- ``gating_output[t, topk_ids[t, j]]`` for
  callers that already hold the probabilities and ids.
* :func:`moe_permute` -- per-expert counts, exclusive offsets and the stable
  expert-major order of the ``T*k`` assignments (``moe_align_block_size``'s
  order, INFERENCE_REPO_CHANGES.md:274-278).
* :func:`expert_token_stats` -- the reference's routing histogram report
  (analysis/moe_regime.py:197-213), counted by the permute kernel.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Tuple

import torch

from . import _lib


def route_topk(logits: torch.Tensor, top_k: int, renormalize: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(topk_ids int32 [T, k], topk_weights fp32 [T, k])`` from router logits ``[..., E]``.

    ids are ordered by descending probability, ties to the lower expert id;
    weights are the fp32 softmax probabilities, renormalized over the k
    chosen experts when ``renormalize``.
    """
    if logits.dim() < 1:
        raise ValueError("router logits need a trailing expert axis")
    E = logits.shape[-1]
    if not 1 <= top_k <= E:
        raise ValueError(f"top_k must lie in [1, {E}], got {top_k}")
    x = logits.reshape(-1, E)
    if x.dtype not in _lib.DTYPE_CODES:
        x = x.to(torch.float32)
    x = x.contiguous()
    device = _lib.require_hip(x)
    T = x.shape[0]
    ids = torch.empty(T, top_k, dtype=torch.int32, device=device)
    weights = torch.empty(T, top_k, dtype=torch.float32, device=device)
    if T:
        lib = _lib.load()
        with torch.cuda.device(device):
            rc = lib.lq_route_topk(_lib.ptr(x), _lib.dtype_code(x.dtype, "logits"), T, E, top_k, int(renormalize),
                                   _lib.ptr(ids), _lib.ptr(weights), _lib.stream(device))
        _lib.check(rc, "route_topk")
    return ids, weights


def route_gemm_topk(hidden_states: torch.Tensor, gate_weight: torch.Tensor, top_k: int,
                    renormalize: bool = False, return_logits: bool = False):
    """Router GEMM + top-k in one kernel: ``(ids, weights[, logits])`` for ``hidden_states [..., H]``.

    ``logits = bf16(x . gate_weight^T)`` (``block.gate(x_flat)``, a bias-free bf16
    nn.Linear, fp32 accumulation), then the route_topk routing of those logits
    (trajectory/llada.py:228-234).  ``gate_weight`` is ``[E, H]`` bf16, E <= 64.
    """
    H = hidden_states.shape[-1]
    x = hidden_states.reshape(-1, H)
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    x = x.contiguous()
    wg = gate_weight.to(torch.bfloat16).contiguous()
    if wg.dim() != 2 or wg.shape[1] != H:
        raise ValueError(f"gate_weight must be [experts, {H}], got {tuple(gate_weight.shape)}")
    E = wg.shape[0]
    if not 1 <= top_k <= E:
        raise ValueError(f"top_k must lie in [1, {E}], got {top_k}")
    device = _lib.require_hip(x, wg)
    T = x.shape[0]
    ids = torch.empty(T, top_k, dtype=torch.int32, device=device)
    weights = torch.empty(T, top_k, dtype=torch.float32, device=device)
    logits = torch.empty(T, E, dtype=torch.bfloat16, device=device) if return_logits else None
    if T:
        lib = _lib.load()
        with torch.cuda.device(device):
            rc = lib.lq_route_gemm_topk(_lib.ptr(x), _lib.ptr(wg), T, H, E, top_k, int(renormalize), _lib.ptr(ids),
                                        _lib.ptr(weights), _lib.ptr(logits), _lib.stream(device))
        _lib.check(rc, "route_gemm_topk")
    return (ids, weights, logits) if return_logits else (ids, weights)


def gather_topk_weights(gating_output: torch.Tensor, topk_ids: torch.Tensor,
                        renormalize: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """``(ids int32, weights fp32)`` with ``weights[t, j] = gating_output[t, topk_ids[t, j]]``."""
    T, E = gating_output.shape
    if topk_ids.dim() != 2 or topk_ids.shape[0] != T:
        raise ValueError(f"topk_ids must be [tokens, top_k] with {T} tokens, got {tuple(topk_ids.shape)}")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"topk_ids must be int32 or int64, got {topk_ids.dtype}")
    k = topk_ids.shape[1]
    probs = gating_output.to(torch.float32).contiguous()
    ids_in = topk_ids.contiguous()
    device = _lib.require_hip(probs, ids_in)
    ids = torch.empty(T, k, dtype=torch.int32, device=device)
    weights = torch.empty(T, k, dtype=torch.float32, device=device)
    if T:
        lib = _lib.load()
        with torch.cuda.device(device):
            rc = lib.lq_gather_topk_weights(_lib.ptr(probs), _lib.ptr(ids_in), int(ids_in.dtype == torch.int64), T, E,
                                            k, int(renormalize), _lib.ptr(ids), _lib.ptr(weights),
                                            _lib.stream(device))
        _lib.check(rc, "gather_topk_weights")
    return ids, weights


def moe_permute(topk_ids: torch.Tensor, num_experts: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``(counts [E], offsets [E+1], sorted [T*k])`` int32 for ``topk_ids [T, k]``.

    ``sorted`` lists the flat assignment ids ``t*k + j`` grouped by expert,
    ascending within an expert.  Ids outside ``[0, E)`` are not routed.
    """
    if topk_ids.dim() != 2:
        raise ValueError(f"topk_ids must be [tokens, top_k], got {tuple(topk_ids.shape)}")
    ids = topk_ids.to(torch.int32).contiguous()
    device = _lib.require_hip(ids)
    T, k = ids.shape
    counts = torch.empty(num_experts, dtype=torch.int32, device=device)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=device)
    sorted_ = torch.empty(T * k, dtype=torch.int32, device=device)
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.lq_moe_permute(_lib.ptr(ids), T, k, num_experts, _lib.ptr(counts), _lib.ptr(offsets),
                                _lib.ptr(sorted_), _lib.stream(device))
    _lib.check(rc, "moe_permute")
    return counts, offsets, sorted_


@dataclass
class ExpertTokenStats:
    """Rows per expert from real routing (analysis/moe_regime.py:152-213)."""

    tokens: int
    top_k: int
    num_experts: int
    counts: List[int] = field(default_factory=list)

    @property
    def active_experts(self) -> int:
        return sum(1 for c in self.counts if c > 0)

    @property
    def mean(self) -> float:
        """Rows per counted expert (0.0 for an empty histogram)."""
        return sum(self.counts) / len(self.counts) if self.counts else 0.0

    @property
    def imbalance(self) -> float:
        """Busiest expert's rows over the mean; 1.0 (balanced) when nothing was routed."""
        m = self.mean
        return max(self.counts) / m if m else 1.0

    def percentile(self, p: float) -> float:
        ordered = sorted(self.counts)
        if not ordered:
            return 0.0
        idx = min(len(ordered) - 1, max(0, int(round(p / 100.0 * (len(ordered) - 1)))))
        return float(ordered[idx])

    def to_dict(self) -> dict:
        """The reference's report keys and rounding (analysis/moe_regime.py:186-199)."""
        lo, hi = (min(self.counts), max(self.counts)) if self.counts else (0, 0)
        return {
            "tokens": self.tokens,
            "top_k": self.top_k,
            "num_experts": self.num_experts,
            "active_experts": self.active_experts,
            "min": lo,
            "p50": self.percentile(50),
            "mean": round(self.mean, 2),
            "p90": self.percentile(90),
            "p99": self.percentile(99),
            "max": hi,
            "imbalance_max_over_mean": round(self.imbalance, 3),
        }


def expert_token_stats(topk_ids: torch.Tensor, num_experts: int) -> ExpertTokenStats:
    """Per-expert row counts of ``topk_ids [tokens, top_k]``, counted on the GPU."""
    if topk_ids.dim() != 2:
        raise ValueError(f"topk_ids must be [tokens, top_k], got {tuple(topk_ids.shape)}")
    counts, _, _ = moe_permute(topk_ids, num_experts)
    return ExpertTokenStats(tokens=topk_ids.shape[0], top_k=topk_ids.shape[1], num_experts=num_experts,
                            counts=counts.cpu().tolist())
