"""The reference's PACKED expert layer on the CPU with torch (dequantize, then matmul).

TEST INFRASTRUCTURE ONLY: the timed CPU baseline of ``bench.py`` (its
``cpu_baseline`` leg) and a cross-check in ``tests/``.  Never imported by the
product package.

It restates, op for op, what one LLaDA_Quant v0.2.0 PACKED layer costs on
the CPU:

* ``block.w1`` / ``block.w2`` dequantize the WHOLE packed tensors on every
  access (runtime/moe.py:199-216): ``unpack_int4`` with int8 shifts
  (algorithms/symmetric.py:316-346), then ``(q.float() * s.float()).to(bf16)``
  per group (:272-293);
* routing ``softmax(logits, fp32).topk(k)`` (trajectory/llada.py:228-234);
* ``fused_moe`` as per-expert gathered BF16 matmuls with the SiLU-epilogue op
  order (INFERENCE_REPO_CHANGES.md:296-309): g, u rounded to bf16, silu in
  fp32 rounded to bf16, bf16 product, then ``act @ W2[e]^T`` scaled by the
  routed weight and summed over the k slots.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    low = (packed << 4) >> 4
    high = packed >> 4
    out = torch.empty(*packed.shape[:-1], packed.shape[-1] * 2, dtype=torch.int8)
    out[..., 0::2] = low
    out[..., 1::2] = high
    return out


def dequantize(q: torch.Tensor, scale: torch.Tensor, bits: int, group_size: int) -> torch.Tensor:
    if bits == 4:
        q = unpack_int4(q)
    k = q.shape[-1]
    if group_size == -1 or k % group_size != 0:
        return (q.to(torch.float32) * scale.to(torch.float32)).to(torch.bfloat16)
    qg = q.reshape(*q.shape[:-1], k // group_size, group_size)
    s = scale.reshape(*q.shape[:-1], k // group_size, 1)
    return (qg.to(torch.float32) * s.to(torch.float32)).reshape(q.shape).to(torch.bfloat16)


def packed_layer(x, logits, q1, s1, q2, s2, bits, group_size, top_k, renormalize=False):
    """One PACKED MoE layer forward; returns (out bf16 [T, H], topk_ids [T, k])."""
    w1 = dequantize(q1, s1, bits, group_size)
    w2 = dequantize(q2, s2, bits, group_size)
    I = w2.shape[-1]
    probs = F.softmax(logits, dim=-1, dtype=torch.float32)
    topk = probs.topk(top_k, dim=-1)
    weights = topk.values
    if renormalize:
        weights = weights / weights.sum(dim=-1, keepdim=True)
    ids = topk.indices
    out = torch.zeros(x.shape[0], x.shape[1], dtype=torch.float32)
    flat = ids.reshape(-1)
    order = torch.argsort(flat, stable=True)
    counts = torch.bincount(flat, minlength=w1.shape[0]).tolist()
    start = 0
    for e, c in enumerate(counts):
        if c == 0:
            continue
        sel = order[start:start + c]
        start += c
        tok = sel // top_k
        xe = x[tok]
        g = xe @ w1[e, :I].T
        u = xe @ w1[e, I:].T
        act = (F.silu(g.float()).to(torch.bfloat16).float() * u.float()).to(torch.bfloat16)
        y = (act @ w2[e].T).float()
        out.index_add_(0, tok, y * weights.reshape(-1)[sel].unsqueeze(1))
    return out.to(torch.bfloat16), ids
