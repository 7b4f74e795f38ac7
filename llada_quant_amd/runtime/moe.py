"""Quantized MoE expert weights and their two residency modes.

Drop-in for ``LLaDA_Quant.runtime.moe`` (v0.2.0, ``src/LLaDA_Quant/runtime/moe.py``).
The fused layout is the one ``TritonFusedMoEBlock`` uses::

    w1: [experts, 2 * intermediate, hidden]   gate rows [:I], up rows [I:]
    w2: [experts, hidden, intermediate]

``ExecutionMode.REFERENCE`` keeps dequantized Parameters next to the packed
buffers.  ``ExecutionMode.PACKED`` deletes the Parameters; ``block.w1`` /
``block.w2`` become read-only properties of a generated subclass, exactly as
in the reference (moe.py:243-286).

What the property returns is the one deliberate difference: a
:class:`PackedExpertTensor`, a tensor of the logical shape and compute dtype
that *holds the packed buffers instead of BF16 data*.  Any torch operation on
it dequantizes through the HIP kernel first (bit-exact to the reference's
``dequantize_tensor``), and every access builds a fresh object, so code that
reads ``block.w1`` sees what the reference returns.  :func:`fused_moe`
recognises it and hands the packed codes and scales straight to the grouped
GEMM, so in the hot path the BF16 copy never exists.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Tuple

import torch
import torch.nn as nn
from torch.utils._pytree import tree_map

from ..algorithms.symmetric import QuantResult, dequantize_tensor, quantize_tensor

W1 = "w1"
W2 = "w2"
EXPERT_PARAM_NAMES = (W1, W2)
PACKED_BUFFERS = ("_qw1", "_sw1", "_qw2", "_sw2")
QUANT_META_ATTR = "_llada_quant_meta"


@dataclass
class QuantExpertWeights:
    """Packed codes + scales for one MoE layer's ``w1`` and ``w2`` (moe.py:48-79)."""

    w1: QuantResult
    w2: QuantResult

    @classmethod
    def quantize(
        cls,
        w1: torch.Tensor,
        w2: torch.Tensor,
        bits: int = 8,
        group_size: int = 128,
        scale_dtype: torch.dtype = torch.float32,
        scale_search: str = "amax",
        search_grid: int = 24,
    ) -> "QuantExpertWeights":
        kw = dict(bits=bits, group_size=group_size, scale_dtype=scale_dtype, scale_search=scale_search,
                  search_grid=search_grid)
        return cls(w1=quantize_tensor(w1, **kw), w2=quantize_tensor(w2, **kw))

    def dequantize(self, dtype: torch.dtype = torch.bfloat16) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.w1.dequantize(dtype=dtype), self.w2.dequantize(dtype=dtype)

    def storage_bytes(self) -> int:
        return self.w1.storage_bytes() + self.w2.storage_bytes()


def quant_result_from_buffers(q: torch.Tensor, scale: torch.Tensor, bits: int) -> QuantResult:
    """Rebuild a :class:`QuantResult` from stored tensors (moe.py:82-102).

    The group length is derived from the scale tensor, never from a config:
    the quantizer falls back to one group per row when the configured size
    does not divide K, and trusting the config would regroup silently.
    """
    packed = bits == 4
    k_logical = q.shape[-1] * (2 if packed else 1)
    num_groups = scale.shape[-1] if scale.dim() else 1
    group_size = -1 if num_groups <= 1 else k_logical // num_groups
    return QuantResult(q=q, scale=scale, bits=bits, group_size=group_size, packed=packed,
                       logical_shape=tuple(list(q.shape[:-1]) + [k_logical]))


def quantize_fused_experts(
    w1: torch.Tensor,
    w2: torch.Tensor,
    bits: int = 8,
    group_size: int = 128,
    scale_dtype: torch.dtype = torch.float32,
    scale_search: str = "amax",
    search_grid: int = 24,
) -> QuantExpertWeights:
    """Quantize a fused ``w1``/``w2`` pair (moe.py:105-118)."""
    return QuantExpertWeights.quantize(w1, w2, bits=bits, group_size=group_size, scale_dtype=scale_dtype,
                                       scale_search=scale_search, search_grid=search_grid)


def materialize_expert_params(
    module: nn.Module,
    weights: QuantExpertWeights,
    compute_dtype: torch.dtype = torch.bfloat16,
) -> None:
    """REFERENCE mode: write dequantized weights into the live Parameters (moe.py:121-139)."""
    if is_packed_expert_block(module):
        raise RuntimeError(
            "materialize_expert_params() called on a PACKED block: w1/w2 are "
            "derived from the packed buffers and cannot be assigned. Use "
            "ExecutionMode.REFERENCE if you need writable BF16 Parameters."
        )
    w1, w2 = weights.dequantize(dtype=compute_dtype)
    module.w1.data.copy_(w1)
    module.w2.data.copy_(w2)


# ---------------------------------------------------------------------------
# the packed weight handle returned by block.w1 / block.w2
# ---------------------------------------------------------------------------


class PackedExpertTensor(torch.Tensor):
    """Logical ``[E, N, K]`` compute-dtype tensor backed by packed codes.

    Shape, dtype and device queries answer from metadata.  Every other torch
    operation first dequantizes (``materialize()``, one HIP kernel, bit-exact
    to ``dequantize_tensor``) and runs on the result, so the object behaves
    like the fresh BF16 tensor the reference property returns.  It has no
    storage of its own: ``data_ptr()`` is unavailable, by design.
    """

    qweight: torch.Tensor
    scale: torch.Tensor
    bits: int
    group_size: int
    packed: bool

    @staticmethod
    def __new__(cls, q: torch.Tensor, scale: torch.Tensor, bits: int, group_size: int, packed: bool,
                logical_shape: Tuple[int, ...], dtype: torch.dtype):
        t = torch.Tensor._make_wrapper_subclass(cls, tuple(logical_shape), dtype=dtype, device=q.device,
                                                requires_grad=False)
        t.qweight = q
        t.scale = scale
        t.bits = bits
        t.group_size = group_size
        t.packed = packed
        return t

    def __init__(self, *args, **kwargs) -> None:  # everything is set in __new__
        super().__init__()

    def materialize(self) -> torch.Tensor:
        """The dequantized tensor (fresh memory on every call)."""
        return dequantize_tensor(self.qweight, self.scale, self.bits, self.group_size, dtype=self.dtype,
                                 packed=self.packed)

    def quant_result(self) -> QuantResult:
        return QuantResult(q=self.qweight, scale=self.scale, bits=self.bits, group_size=self.group_size,
                           packed=self.packed, logical_shape=tuple(self.shape))

    __torch_function__ = torch._C._disabled_torch_function_impl

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        def unwrap(x):
            return x.materialize() if isinstance(x, PackedExpertTensor) else x

        return func(*tree_map(unwrap, args), **tree_map(unwrap, kwargs or {}))

    def __repr__(self) -> str:
        return (f"PackedExpertTensor(shape={tuple(self.shape)}, dtype={self.dtype}, device={self.device}, "
                f"bits={self.bits}, group_size={self.group_size}, packed={self.packed})")


# ---------------------------------------------------------------------------
# PACKED residency (moe.py:147-301)
# ---------------------------------------------------------------------------


def attach_packed_buffers(
    block: nn.Module,
    weights: QuantExpertWeights,
    compute_dtype: torch.dtype,
    compile_dequant: bool = False,
) -> None:
    """Register ``_qw1``/``_sw1``/``_qw2``/``_sw2`` and the metadata to read them.

    ``compile_dequant`` is kept in the metadata for compatibility; the HIP
    dequant kernel is already one fused pass, so it changes nothing.
    """
    block.register_buffer("_qw1", weights.w1.q, persistent=True)
    block.register_buffer("_sw1", weights.w1.scale, persistent=True)
    block.register_buffer("_qw2", weights.w2.q, persistent=True)
    block.register_buffer("_sw2", weights.w2.scale, persistent=True)
    setattr(block, QUANT_META_ATTR, {
        "bits": weights.w1.bits,
        "group_size": weights.w1.group_size,
        "packed": weights.w1.packed,
        "compute_dtype": compute_dtype,
        "compile_dequant": compile_dequant,
        "logical_shape": {W1: weights.w1.logical_shape, W2: weights.w2.logical_shape},
    })


def _packed_expert_weight(self: nn.Module, which: str) -> PackedExpertTensor:
    meta = getattr(self, QUANT_META_ATTR, None)
    if meta is None:
        raise RuntimeError(
            f"{type(self).__name__}.{which} is served from packed buffers but "
            f"{QUANT_META_ATTR} is missing. Reload through "
            "load_quantized_weights() so the quantization config is applied."
        )
    suffix = which[-1]
    q = getattr(self, f"_qw{suffix}")
    scale = getattr(self, f"_sw{suffix}")
    packed = bool(meta["packed"])
    k = q.shape[-1] * (2 if packed else 1)
    logical = tuple(meta.get("logical_shape", {}).get(which, ())) or (*q.shape[:-1], k)
    return PackedExpertTensor(q, scale, int(meta["bits"]), int(meta["group_size"]), packed, logical,
                              meta["compute_dtype"])


#: In-place writers of w1/w2 that PACKED mode turns into loud failures
#: (moe.py:219-240): their write would land in a temporary and vanish.
WEIGHT_MUTATING_METHODS = ("load_state_dict_from_unfused",)


def _blocked_method(name: str):
    def blocked(self, *args, **kwargs):
        raise RuntimeError(
            f"{type(self).__mro__[1].__name__}.{name}() writes into w1/w2 in place, "
            "but this block is quantized in PACKED mode where those are derived "
            "from packed buffers — the write would be silently discarded.\n"
            "Load the weights first, then quantize:\n"
            f"    block.{name}(...)\n"
            "    quantize_model(model, config)"
        )

    blocked.__name__ = name
    return blocked


_PACKED_CLASS_CACHE: Dict[type, type] = {}


def _packed_class(cls: type) -> type:
    """Subclass of ``cls`` whose ``w1``/``w2`` are served from packed buffers (cached per class)."""
    if getattr(cls, "_llada_quant_packed", False):
        return cls
    cached = _PACKED_CLASS_CACHE.get(cls)
    if cached is not None:
        return cached
    namespace = {
        "_llada_quant_packed": True,
        "_packed_expert_weight": _packed_expert_weight,
        W1: property(lambda self: self._packed_expert_weight(W1)),
        W2: property(lambda self: self._packed_expert_weight(W2)),
        "__doc__": f"{cls.__name__} with w1/w2 served from packed integer buffers.",
    }
    for method in WEIGHT_MUTATING_METHODS:
        if hasattr(cls, method):
            namespace[method] = _blocked_method(method)
    generated = type(f"PackedQuant{cls.__name__}", (cls,), namespace)
    _PACKED_CLASS_CACHE[cls] = generated
    return generated


def install_packed_expert_access(block: nn.Module) -> None:
    """Drop the BF16 ``w1``/``w2`` Parameters and serve them from the packed buffers."""
    missing = [name for name in PACKED_BUFFERS if not hasattr(block, name)]
    if missing:
        raise RuntimeError(f"cannot install packed access, missing buffers: {missing}")
    for name in EXPERT_PARAM_NAMES:
        block._parameters.pop(name, None)
    block.__class__ = _packed_class(type(block))


def is_packed_expert_block(module: nn.Module) -> bool:
    """True when ``w1``/``w2`` are derived from packed buffers."""
    return getattr(type(module), "_llada_quant_packed", False)


def expert_storage_bytes(block: nn.Module) -> int:
    """Bytes the packed representation occupies on this block."""
    total = 0
    for name in PACKED_BUFFERS:
        buf = getattr(block, name, None)
        if buf is not None:
            total += buf.numel() * buf.element_size()
    return total
