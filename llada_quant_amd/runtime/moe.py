"""Quantized MoE expert weights and their two residency modes.

Drop-in for ``LLaDA_Quant.runtime.moe`` (v0.2.0, ``src/LLaDA_Quant/runtime/moe.py``):
the same names, buffers (``_qw1/_sw1/_qw2/_sw2``), metadata attribute and
error messages.  The fused layout is ``TritonFusedMoEBlock``'s::

    w1: [experts, 2 * intermediate, hidden]   gate rows [:I], up rows [I:]
    w2: [experts, hidden, intermediate]

``ExecutionMode.REFERENCE`` keeps dequantized Parameters next to the packed
buffers.  ``ExecutionMode.PACKED`` removes the Parameters and turns the block
into an instance of a subclass of its own class (made once per class, named
``PackedQuant<Class>``) whose ``w1``/``w2`` are read-only properties.

What those properties return is a :class:`PackedExpertTensor`: a tensor of
the logical shape and compute dtype that holds the packed buffers instead of
BF16 data.  Any torch operation on it dequantizes through the HIP kernel
first (bit-exact to ``dequantize_tensor``), and every access builds a fresh
object, so code reading ``block.w1`` sees what the reference's property
returns; :func:`fused_moe` recognises it and hands the codes and scales to
the grouped GEMMs, so in the hot path the BF16 copy never exists.
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
#: Methods of expert-block classes that write into w1/w2 in place; a PACKED
#: block refuses them (the write would land in a temporary and vanish).
WEIGHT_MUTATING_METHODS = ("load_state_dict_from_unfused",)


@dataclass
class QuantExpertWeights:
    """Codes and scales of one layer's ``w1`` and ``w2`` (runtime/moe.py:48-79)."""

    w1: QuantResult
    w2: QuantResult

    @classmethod
    def quantize(cls, w1: torch.Tensor, w2: torch.Tensor, bits: int = 8, group_size: int = 128,
                 scale_dtype: torch.dtype = torch.float32, scale_search: str = "amax",
                 search_grid: int = 24) -> "QuantExpertWeights":
        settings = dict(bits=bits, group_size=group_size, scale_dtype=scale_dtype, scale_search=scale_search,
                        search_grid=search_grid)
        return cls(*(quantize_tensor(w, **settings) for w in (w1, w2)))

    def results(self) -> Tuple[QuantResult, QuantResult]:
        return self.w1, self.w2

    def dequantize(self, dtype: torch.dtype = torch.bfloat16) -> Tuple[torch.Tensor, torch.Tensor]:
        d1, d2 = (r.dequantize(dtype=dtype) for r in self.results())
        return d1, d2

    def storage_bytes(self) -> int:
        return sum(r.storage_bytes() for r in self.results())


def quant_result_from_buffers(q: torch.Tensor, scale: torch.Tensor, bits: int) -> QuantResult:
    """A :class:`QuantResult` from stored codes and scales alone (runtime/moe.py:82-102).

    The group length comes from the scales: the quantizer falls back to one
    group per row when the requested length does not divide K, so the
    config's length may not be the one the codes were made with.
    """
    packed = bits == 4
    k = q.shape[-1] * 2 if packed else q.shape[-1]
    groups = scale.shape[-1] if scale.dim() > 0 else 1
    return QuantResult(q=q, scale=scale, bits=bits, group_size=k // groups if groups > 1 else -1, packed=packed,
                       logical_shape=(*q.shape[:-1], k))


def quantize_fused_experts(w1: torch.Tensor, w2: torch.Tensor, bits: int = 8, group_size: int = 128,
                           scale_dtype: torch.dtype = torch.float32, scale_search: str = "amax",
                           search_grid: int = 24) -> QuantExpertWeights:
    """Quantize a fused ``w1``/``w2`` pair (runtime/moe.py:105-118)."""
    return QuantExpertWeights.quantize(w1, w2, bits, group_size, scale_dtype, scale_search, search_grid)


def materialize_expert_params(module: nn.Module, weights: QuantExpertWeights,
                              compute_dtype: torch.dtype = torch.bfloat16) -> None:
    """REFERENCE mode: overwrite the live ``w1``/``w2`` Parameters with the dequantized weights."""
    if is_packed_expert_block(module):
        raise RuntimeError(
            "materialize_expert_params() called on a PACKED block: w1/w2 are "
            "derived from the packed buffers and cannot be assigned. Use "
            "ExecutionMode.REFERENCE if you need writable BF16 Parameters."
        )
    for name, value in zip(EXPERT_PARAM_NAMES, weights.dequantize(dtype=compute_dtype)):
        getattr(module, name).data.copy_(value)


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
# PACKED residency
# ---------------------------------------------------------------------------


def attach_packed_buffers(block: nn.Module, weights: QuantExpertWeights, compute_dtype: torch.dtype,
                          compile_dequant: bool = False) -> None:
    """Register the four packed buffers on ``block`` and the metadata that reads them.

    ``compile_dequant`` is recorded for the reference's config round trip;
    the HIP dequant kernel is already one fused pass, so it changes nothing.
    """
    for suffix, result in zip("12", weights.results()):
        block.register_buffer(f"_qw{suffix}", result.q, persistent=True)
        block.register_buffer(f"_sw{suffix}", result.scale, persistent=True)
    meta = {
        "bits": weights.w1.bits,
        "group_size": weights.w1.group_size,
        "packed": weights.w1.packed,
        "compute_dtype": compute_dtype,
        "compile_dequant": compile_dequant,
        "logical_shape": {name: r.logical_shape for name, r in zip(EXPERT_PARAM_NAMES, weights.results())},
    }
    setattr(block, QUANT_META_ATTR, meta)


def _packed_weight(block: nn.Module, which: str) -> PackedExpertTensor:
    """``block.w1`` / ``block.w2`` of a PACKED block: a fresh handle on the packed buffers."""
    meta = getattr(block, QUANT_META_ATTR, None)
    if meta is None:
        raise RuntimeError(
            f"{type(block).__name__}.{which} is served from packed buffers but {QUANT_META_ATTR} is missing. "
            "Reload through load_quantized_weights() so the quantization config is applied."
        )
    q = getattr(block, "_q" + which)
    scale = getattr(block, "_s" + which)
    packed = bool(meta["packed"])
    shape = tuple(meta.get("logical_shape", {}).get(which, ())) or (*q.shape[:-1], q.shape[-1] * (2 if packed else 1))
    return PackedExpertTensor(q, scale, int(meta["bits"]), int(meta["group_size"]), packed, shape,
                              meta["compute_dtype"])


class _PackedExpertAccess:
    """Mixin placed in front of an expert block's own class in PACKED mode."""

    _llada_quant_packed = True
    w1 = property(lambda self: _packed_weight(self, W1), doc="w1 served from _qw1/_sw1 (read-only)")
    w2 = property(lambda self: _packed_weight(self, W2), doc="w2 served from _qw2/_sw2 (read-only)")


def _refuse_in_place_write(method: str):
    def refuse(self, *args, **kwargs):
        base = unpacked_class(type(self)).__name__
        raise RuntimeError(
            f"{base}.{method}() writes into w1/w2 in place, but this block is quantized in PACKED mode "
            "where those are derived from packed buffers — the write would be silently discarded.\n"
            "Load the weights first, then quantize:\n"
            f"    block.{method}(...)\n"
            "    quantize_model(model, config)"
        )

    refuse.__name__ = method
    return refuse


_PACKED_CLASSES: Dict[type, type] = {}


def packed_class_for(cls: type) -> type:
    """The PACKED variant of expert-block class ``cls`` (made once, then reused)."""
    if issubclass(cls, _PackedExpertAccess):
        return cls
    if cls not in _PACKED_CLASSES:
        body = {name: _refuse_in_place_write(name) for name in WEIGHT_MUTATING_METHODS if hasattr(cls, name)}
        body["__doc__"] = f"{cls.__name__} whose w1/w2 are served from packed integer buffers."
        body["_unpacked_class"] = cls
        _PACKED_CLASSES[cls] = type(f"PackedQuant{cls.__name__}", (_PackedExpertAccess, cls), body)
    return _PACKED_CLASSES[cls]


def unpacked_class(cls: type) -> type:
    """The block's own class, also for a PACKED block."""
    return getattr(cls, "_unpacked_class", cls)


def install_packed_expert_access(block: nn.Module) -> None:
    """PACKED residency: drop the BF16 ``w1``/``w2`` Parameters; serve them from the packed buffers.

    Afterwards ``state_dict()`` holds no BF16 copy, every ``block.w1`` read
    is a fresh handle, and assigning ``block.w1`` raises (a property with no
    setter).
    """
    absent = [name for name in PACKED_BUFFERS if not hasattr(block, name)]
    if absent:
        raise RuntimeError(f"cannot install packed access, missing buffers: {absent}")
    for name in EXPERT_PARAM_NAMES:
        block._parameters.pop(name, None)
    block.__class__ = packed_class_for(type(block))


def is_packed_expert_block(module: nn.Module) -> bool:
    """True when ``w1``/``w2`` are derived from packed buffers, not stored."""
    return isinstance(module, _PackedExpertAccess)


def expert_storage_bytes(block: nn.Module) -> int:
    """Bytes of the packed buffers present on this block."""
    return sum(b.numel() * b.element_size() for b in (getattr(block, n, None) for n in PACKED_BUFFERS)
               if b is not None)
