"""``fused_moe`` over packed expert weights: the quantized expert layer in one HIP call.

Drop-in for the inference repository's
``fused_moe(hidden_states, w1, w2, gating_output, topk_ids, fuse_silu=None)``
(INFERENCE_REPO_CHANGES.md:109-111) as ``TritonFusedMoEBlock.forward`` calls
it with ``w1=self.w1, w2=self.w2``.  With a PACKED block those arguments are
:class:`~llada_quant_amd.runtime.moe.PackedExpertTensor` handles, and this
function passes their INT4/INT8 codes and fp32 scales straight to
``lq_moe_forward``: grouped GEMMs that dequantize in registers, the SwiGLU
activation fused into GEMM1 (the ``SILU_EPILOGUE`` op order,
INFERENCE_REPO_CHANGES.md:296-309) and the routed-weight scaling plus top-k
combine fused into GEMM2.  No BF16 copy of a weight is ever written.

``gating_output`` carries the router's softmax probabilities ``[T, E]``; the
routed weight of slot ``(t, j)`` is ``gating_output[t, topk_ids[t, j]]``,
renormalized over the k slots when ``renormalize``.  ``topk_weights`` may be
passed instead.  :func:`moe_layer` runs the router too, from logits.
"""

from __future__ import annotations

from typing import Optional, Tuple, Union

import torch

from ..algorithms.symmetric import QuantResult
from . import _lib
from .moe import PackedExpertTensor
from .routing import gather_topk_weights

PackedWeight = Union[PackedExpertTensor, QuantResult]


def _unpack_weight(w: PackedWeight, name: str) -> QuantResult:
    if isinstance(w, PackedExpertTensor):
        return w.quant_result()
    if isinstance(w, QuantResult):
        return w
    raise TypeError(
        f"fused_moe consumes packed expert weights: pass block.{name} of a PACKED block "
        f"(a PackedExpertTensor) or a QuantResult, got {type(w).__name__}"
    )


def workspace_bytes(tokens: int, hidden: int, intermediate: int, num_experts: int, top_k: int) -> int:
    return int(_lib.load().lq_moe_workspace_bytes(tokens, hidden, intermediate, num_experts, top_k))


def moe_workspace(tokens: int, hidden: int, intermediate: int, num_experts: int, top_k: int,
                  device: torch.device) -> torch.Tensor:
    """A zero-initialised workspace for layers of this shape (reusable across calls on one stream)."""
    return _lib.moe_workspace(workspace_bytes(tokens, hidden, intermediate, num_experts, top_k), device)


def fused_moe_packed(
    x: torch.Tensor,
    w1: QuantResult,
    w2: QuantResult,
    topk_ids: torch.Tensor,
    topk_weights: torch.Tensor,
    out: Optional[torch.Tensor] = None,
    workspace: Optional[torch.Tensor] = None,
    folded_scales: bool = False,
    general_kernel: bool = False,
    wide_kernel: bool = False,
    stream_kernel: bool = False,
    fused_layer: bool = False,
) -> torch.Tensor:
    """The layer on explicit operands: ``x [T, H]`` bf16, int32 ids and fp32 weights ``[T, k]``.

    The matrix cores consume the reference's dequantized BF16 weights
    ``bf16(fp32(q) * s)`` bit for bit.  ``folded_scales`` instead feeds the
    codes as exact integers and multiplies each group's fp32 scale into their
    dot product: cheaper, but without the per-weight BF16 rounding the output
    moves by about the reference tolerance (mean-relative ~5e-3).
    ``general_kernel`` runs the general GEMM kernels even where the streaming
    ones apply, ``wide_kernel`` the wide (matrix-core) ones, which layers with
    at least 32 routed rows per expert on average take by themselves, and
    ``stream_kernel`` the streaming (weight-bandwidth) ones, which smaller
    layers take (same results bit for bit; for comparison).  ``fused_layer``
    runs a small streaming-family layer (E <= 64, T*k <= 2048) as one launch,
    the fused layer kernel, instead of GEMM1, GEMM2 and combine (same bits).  A ``workspace``
    passed in must come from :func:`moe_workspace` (or otherwise start with a
    zero sync region, ``lq_moe_sync_bytes`` bytes); it may be reused by later
    calls on the same stream.
    """
    g1, g2, I = _check_weights(x, w1, w2)
    T, H = x.shape
    E = w1.logical_shape[0]
    k = topk_ids.shape[1]
    if topk_ids.shape[0] != T or topk_weights.shape != topk_ids.shape:
        raise ValueError("topk_ids / topk_weights must be [tokens, top_k]")
    xc = x.contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    wts = topk_weights.to(torch.float32).contiguous()
    q1, s1, q2, s2 = (t.contiguous() for t in (w1.q, w1.scale, w2.q, w2.scale))
    device = _lib.require_hip(xc, ids, wts, q1, s1, q2, s2)
    if out is None:
        out = torch.empty(T, H, dtype=torch.bfloat16, device=device)
    spans = _chunks(T, max_tokens_per_call(H, I, k))
    tc = max(c1 - c0 for c0, c1 in spans)
    ws_need = workspace_bytes(tc, H, I, E, k)
    if workspace is None or workspace.numel() < ws_need:
        workspace = _lib.moe_workspace(ws_need, device)
    flags = (_moe_flags(folded_scales)
             | (_lib.LQ_MOE_GENERAL_KERNEL if general_kernel else 0)
             | (_lib.LQ_MOE_WIDE_KERNEL if wide_kernel else 0)
             | (_lib.LQ_MOE_STREAM_KERNEL if stream_kernel else 0)
             | (_lib.LQ_MOE_FUSED_LAYER if fused_layer else 0))
    if T:
        lib = _lib.load()
        with torch.cuda.device(device):
            for c0, c1 in spans:
                rc = lib.lq_moe_forward(
                    _lib.ptr(xc[c0:c1]), c1 - c0, H, I, E, k, _lib.ptr(q1), _lib.ptr(s1), _lib.ptr(q2), _lib.ptr(s2),
                    w1.bits, g1, g2, flags, _lib.ptr(ids[c0:c1]), _lib.ptr(wts[c0:c1]), _lib.ptr(workspace),
                    workspace.numel(), _lib.ptr(out[c0:c1]), _lib.stream(device),
                )
                _lib.check(rc, "fused_moe")
        _lib.check_status(workspace, "fused_moe")
    return out


def max_tokens_per_call(H: int, I: int, top_k: int) -> int:
    """Largest token count one library call takes.

    The kernels address the per-assignment buffers (bf16 gate / up rows
    [T*k, 2I] and slot outputs [T*k, H]) and x with 32-bit offsets:
    T*k*max(2I, H)*2 must stay below 2^31, T*H*2 below the buffer descriptor
    range, and T <= 2^18.  Larger inputs are split into token chunks by
    fused_moe_packed and moe_layer (a token's output depends only on its own
    row and routing, so the split is exact).
    """
    lim = min((2**31 - 1) // (top_k * max(2 * I, H) * 2), (0x7FFFFFF0 - 1) // (H * 2), 1 << 18)
    return max(lim, 1)


def _chunks(T: int, lim: int):
    """Even token ranges [c0, c1) of at most lim tokens covering [0, T)."""
    n = max(1, -(-T // lim))
    return [(i * T // n, (i + 1) * T // n) for i in range(n)]


def _moe_flags(folded_scales: bool) -> int:
    return _lib.LQ_MOE_FOLDED_SCALES if folded_scales else 0


def _check_weights(x: torch.Tensor, w1: QuantResult, w2: QuantResult):
    """Validate x and the packed operands on the host; returns (G1, G2, I).

    Every operand shape is checked here because the kernels trust them.
    """
    if x.dim() != 2:
        raise ValueError(f"x must be [tokens, hidden], got {tuple(x.shape)}")
    if x.dtype != torch.bfloat16:
        raise ValueError(f"fused_moe computes in bfloat16; hidden_states are {x.dtype}")
    T, H = x.shape
    if len(w1.logical_shape) != 3 or len(w2.logical_shape) != 3:
        raise ValueError("w1 and w2 must be [experts, 2*intermediate, hidden] and [experts, hidden, intermediate]")
    E, two_i, h1 = w1.logical_shape
    E2, h2, I = w2.logical_shape
    if E != E2 or h1 != H or h2 != H or two_i != 2 * I:
        raise ValueError(
            f"inconsistent shapes: x {tuple(x.shape)}, w1 {tuple(w1.logical_shape)}, w2 {tuple(w2.logical_shape)}"
        )
    if w1.bits != w2.bits or w1.packed != w2.packed or w1.packed != (w1.bits == 4):
        raise ValueError("w1 and w2 must share bits, with INT4 packed two per byte")
    if w1.scale.dtype != torch.float32 or w2.scale.dtype != torch.float32:
        raise NotImplementedError("fused_moe reads float32 scales (QuantConfig.scale_dtype='float32')")
    # every operand shape is checked here: the kernels trust them
    g1 = w1.group_size if (w1.group_size != -1 and H % w1.group_size == 0) else H
    g2 = w2.group_size if (w2.group_size != -1 and I % w2.group_size == 0) else I
    kb = 2 if w1.packed else 1
    expect = {
        "w1 codes": (tuple(w1.q.shape), (E, 2 * I, H // kb)),
        "w1 scales": (tuple(w1.scale.shape), (E, 2 * I, H // g1)),
        "w2 codes": (tuple(w2.q.shape), (E, H, I // kb)),
        "w2 scales": (tuple(w2.scale.shape), (E, H, I // g2)),
    }
    for what, (got, want) in expect.items():
        if got != want:
            raise ValueError(f"{what} have shape {got}, expected {want}")
    if w1.q.dtype != torch.int8 or w2.q.dtype != torch.int8:
        raise ValueError("packed expert codes must be int8")
    return g1, g2, I


def fused_moe(
    hidden_states: torch.Tensor,
    w1: PackedWeight,
    w2: PackedWeight,
    gating_output: Optional[torch.Tensor],
    topk_ids: torch.Tensor,
    fuse_silu: Optional[bool] = None,
    *,
    renormalize: bool = False,
    topk_weights: Optional[torch.Tensor] = None,
    folded_scales: bool = False,
) -> torch.Tensor:
    """Quantized MoE layer output ``[..., H]`` (bf16) for ``hidden_states [..., H]``.

    ``fuse_silu`` is accepted for signature compatibility: the activation is
    always applied in GEMM1's epilogue with the unfused path's rounding, which
    the reference documents as bit-identical to the unfused chain.
    """
    del fuse_silu
    q1 = _unpack_weight(w1, "w1")
    q2 = _unpack_weight(w2, "w2")
    H = hidden_states.shape[-1]
    x = hidden_states.reshape(-1, H)
    if topk_ids.dim() != 2 or topk_ids.shape[0] != x.shape[0]:
        raise ValueError(f"topk_ids must be [tokens, top_k] with {x.shape[0]} tokens, got {tuple(topk_ids.shape)}")
    if topk_weights is None:
        if gating_output is None:
            raise ValueError("fused_moe needs gating_output (softmax probabilities) or topk_weights")
        ids, weights = gather_topk_weights(gating_output.reshape(x.shape[0], -1), topk_ids, renormalize)
    else:
        ids, weights = topk_ids, topk_weights
    out = fused_moe_packed(x, q1, q2, ids, weights, folded_scales=folded_scales)
    return out.reshape(hidden_states.shape)


def moe_layer(
    hidden_states: torch.Tensor,
    router_logits: torch.Tensor,
    w1: PackedWeight,
    w2: PackedWeight,
    top_k: int,
    renormalize: bool = False,
    folded_scales: bool = False,
    fused_layer: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Router + quantized experts in one library call: ``(output [..., H], topk_ids [T, k] int32)``.

    ``router_logits [..., E]`` are the gate's outputs; routing is
    softmax(fp32) -> top-k (descending probability, ties to the lower id),
    weights renormalized over the k experts when ``renormalize``.
    ``fused_layer``: a small streaming-family layer runs as one launch, which
    also routes when T <= 64 (same results).
    """
    q1 = _unpack_weight(w1, "w1")
    q2 = _unpack_weight(w2, "w2")
    H = hidden_states.shape[-1]
    x = hidden_states.reshape(-1, H)
    T = x.shape[0]
    E = q1.logical_shape[0]
    logits = router_logits.reshape(T, -1)
    if logits.shape[1] != E:
        raise ValueError(f"router_logits have {logits.shape[1]} experts, the weights {E}")
    if not 1 <= top_k <= E:
        raise ValueError(f"top_k must lie in [1, {E}], got {top_k}")
    if logits.dtype not in _lib.DTYPE_CODES:
        logits = logits.to(torch.float32)
    logits = logits.contiguous()
    # shape/dtype validation of the weights, shared with fused_moe_packed
    g1, g2, I = _check_weights(x, q1, q2)
    xc = x.contiguous()
    q1c, s1, q2c, s2 = (t.contiguous() for t in (q1.q, q1.scale, q2.q, q2.scale))
    device = _lib.require_hip(xc, logits, q1c, s1, q2c, s2)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=device)
    ids = torch.empty(T, top_k, dtype=torch.int32, device=device)
    spans = _chunks(T, max_tokens_per_call(H, I, top_k))
    tc = max(c1 - c0 for c0, c1 in spans)
    workspace = _lib.moe_workspace(workspace_bytes(tc, H, I, E, top_k), device)
    if T:
        lib = _lib.load()
        code = _lib.dtype_code(logits.dtype, "router_logits")
        with torch.cuda.device(device):
            for c0, c1 in spans:
                rc = lib.lq_moe_layer(
                    _lib.ptr(xc[c0:c1]), _lib.ptr(logits[c0:c1]), code, c1 - c0, H, I, E, top_k, int(renormalize),
                    _lib.ptr(q1c), _lib.ptr(s1), _lib.ptr(q2c), _lib.ptr(s2), q1.bits, g1, g2,
                    _moe_flags(folded_scales) | (_lib.LQ_MOE_FUSED_LAYER if fused_layer else 0),
                    _lib.ptr(workspace), workspace.numel(), _lib.ptr(out[c0:c1]),
                    _lib.ptr(ids[c0:c1]), _lib.stream(device),
                )
                _lib.check(rc, "moe_layer")
        _lib.check_status(workspace, "moe_layer")
    return out.reshape(hidden_states.shape), ids
