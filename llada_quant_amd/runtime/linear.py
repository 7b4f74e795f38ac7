"""QuantLinear: the packed W8A16 / W4A16 replacement for ``nn.Linear`` on MI355X.

Mirrors the reference module (``runtime/linear.py:29-131``): the same
constructor arguments, ``qweight`` ``[out, in]`` int8 (``[out, in // 2]``
packed at 4 bits) and ``scale`` ``[out, groups]`` buffers, ``from_linear``,
``dequantize_weight``, ``storage_bytes`` and ``forward``.  The reference's
forward dequantizes the whole weight to BF16 on every call and runs
``F.linear``; here ``forward`` is one library call (``lq_quant_linear``) whose
GEMM reads the packed codes and scales straight from HBM and feeds the
matrix cores the reference's dequantized weight ``bf16(fp32(q) * s)`` bit for
bit, accumulating in fp32 and rounding the product to bf16 once, as
``F.linear`` in bf16 does.  No BF16 copy of the weight exists.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from ..algorithms.symmetric import QuantResult, dequantize_tensor, quantize_tensor, validate_int4_layout
from . import _lib


def linear_workspace_bytes(M: int, in_features: int, out_features: int) -> int:
    """Workspace bytes lq_quant_linear needs for M rows."""
    return int(_lib.load().lq_linear_workspace_bytes(M, in_features, out_features))


def quant_linear(
    x: torch.Tensor,
    qweight: torch.Tensor,
    scale: torch.Tensor,
    bits: int,
    group_size: int,
    *,
    wide_kernel: bool = False,
    general_kernel: bool = False,
) -> torch.Tensor:
    """``bf16(x . W^T)`` for packed ``W`` (``[..., in] -> [..., out]``), fp32 accumulation.

    ``wide_kernel`` / ``general_kernel`` force one GEMM family (for
    comparison; each is deterministic): by themselves, 128 rows or more take
    the wide kernels where ``out % 256 == 0`` and ``in % 256 == 0``, up to 16
    rows (32 with at most 8 K slices) a one-launch kernel with the general
    family's bits, and the rows between the general family.
    """
    if bits not in (8, 4):
        raise ValueError(f"bits must be 8 or 4, got {bits}")
    if qweight.dtype != torch.int8:
        raise ValueError("qweight must be int8")
    if scale.dtype != torch.float32:
        raise NotImplementedError("quant_linear reads float32 scales (scale_dtype=torch.float32)")
    N = qweight.shape[0]
    K = qweight.shape[1] * (2 if bits == 4 else 1)
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} input features, the weight {K}")
    g = group_size if (group_size != -1 and K % group_size == 0) else K
    if tuple(scale.shape) != (N, K // g):
        raise ValueError(f"scale has shape {tuple(scale.shape)}, expected {(N, K // g)}")
    xc = x.reshape(-1, K).to(torch.bfloat16).contiguous()
    M = xc.shape[0]
    q = qweight.contiguous()
    s = scale.contiguous()
    device = _lib.require_hip(xc, q, s)
    out = torch.empty(M, N, dtype=torch.bfloat16, device=device)
    if M:
        ws = torch.empty(max(linear_workspace_bytes(M, K, N), 1), dtype=torch.uint8, device=device)
        flags = (_lib.LQ_MOE_WIDE_KERNEL if wide_kernel else 0) | (_lib.LQ_MOE_GENERAL_KERNEL if general_kernel else 0)
        lib = _lib.load()
        with torch.cuda.device(device):
            rc = lib.lq_quant_linear(_lib.ptr(xc), M, K, N, _lib.ptr(q), _lib.ptr(s), bits, g, flags, _lib.ptr(ws),
                                     ws.numel(), _lib.ptr(out), _lib.stream(device))
        _lib.check(rc, "quant_linear")
    return out.reshape(*x.shape[:-1], N)


class QuantLinear(nn.Module):
    """Quantized replacement for ``nn.Linear`` with identical call semantics (runtime/linear.py:29-131)."""

    def __init__(
        self,
        in_features: int,
        out_features: int,
        bits: int = 8,
        group_size: int = 128,
        compute_dtype: torch.dtype = torch.bfloat16,
        bias: bool = False,
        scale_dtype: torch.dtype = torch.float32,
    ) -> None:
        super().__init__()
        if bits not in (8, 4):
            raise ValueError(f"bits must be 8 or 4, got {bits}")
        if bits == 4:
            validate_int4_layout((out_features, in_features), group_size)
        if compute_dtype != torch.bfloat16:
            raise NotImplementedError("the packed GEMM computes in bfloat16 (compute_dtype=torch.bfloat16)")
        self.in_features = in_features
        self.out_features = out_features
        self.bits = bits
        self.group_size = group_size
        self.compute_dtype = compute_dtype
        self.packed = bits == 4
        stored_cols = in_features // 2 if self.packed else in_features
        self.register_buffer("qweight", torch.empty(out_features, stored_cols, dtype=torch.int8))
        self.register_buffer("scale", torch.empty(out_features, self._num_groups(), dtype=scale_dtype))
        if bias:
            self.register_buffer("bias", torch.zeros(out_features, dtype=compute_dtype))
        else:
            self.register_buffer("bias", None)

    def _num_groups(self) -> int:
        if self.group_size == -1 or self.in_features % self.group_size != 0:
            return 1
        return self.in_features // self.group_size

    @classmethod
    def from_linear(
        cls,
        linear: nn.Linear,
        bits: int = 8,
        group_size: int = 128,
        compute_dtype: torch.dtype = torch.bfloat16,
        scale_search: str = "amax",
        search_grid: int = 24,
    ) -> "QuantLinear":
        """Quantize an ``nn.Linear`` (its weight on the GPU) with the GPU quantizer."""
        w = linear.weight.detach().to(torch.float32)
        q: QuantResult = quantize_tensor(w, bits=bits, group_size=group_size, scale_search=scale_search,
                                         search_grid=search_grid)
        out = cls(in_features=linear.in_features, out_features=linear.out_features, bits=bits,
                  group_size=group_size, compute_dtype=compute_dtype, bias=linear.bias is not None)
        out = out.to(w.device)
        out.qweight.copy_(q.q)
        out.scale.copy_(q.scale)
        if linear.bias is not None:
            out.bias.copy_(linear.bias.detach())
        return out

    def dequantize_weight(self) -> torch.Tensor:
        return dequantize_tensor(self.qweight, self.scale, self.bits, self.group_size, dtype=self.compute_dtype,
                                 packed=self.packed)

    def storage_bytes(self) -> int:
        """Resident bytes of this module's weight representation."""
        total = self.qweight.numel() * self.qweight.element_size()
        total += self.scale.numel() * self.scale.element_size()
        if self.bias is not None:
            total += self.bias.numel() * self.bias.element_size()
        return total

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bits={self.bits}, group_size={self.group_size}, packed={self.packed}")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = quant_linear(x.to(self.compute_dtype), self.qweight, self.scale, self.bits, self.group_size)
        if self.bias is not None:
            out = out + self.bias
        return out
