"""LLaDA-MoE adapter: find fused expert blocks by their shapes, quantize them, restore them.

Drop-in for ``LLaDA_Quant.adapters.llada_moe`` (v0.2.0): same functions and
records.  A module is a fused expert block of ``TritonFusedMoEBlock``'s layout
when its ``w1`` and ``w2`` are 3-D tensors with

    w1 [E, 2I, H] and w2 [E, H, I]:  one expert count E, one hidden size H,
    and w1 twice as many rows as w2 has columns

held as Parameters (unquantized) or served from packed buffers (PACKED).
Names play no part, so a block is found whatever it is called.
Quantization runs on the GPU that holds the block's weights, through the
HIP quantizer.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterator, List, Optional, Tuple

import torch
import torch.nn as nn

from ..config import ExecutionMode, QuantConfig, is_excluded
from ..formats.manifest import TargetedModule
from ..runtime.moe import (
    EXPERT_PARAM_NAMES,
    PACKED_BUFFERS,
    QuantExpertWeights,
    attach_packed_buffers,
    install_packed_expert_access,
    is_packed_expert_block,
    materialize_expert_params,
    quant_result_from_buffers,
    unpacked_class,
)


@dataclass(frozen=True)
class ExpertBlockShape:
    """Expert count, hidden size and intermediate size of a fused expert block."""

    num_experts: int
    hidden: int
    intermediate: int

    @property
    def numel(self) -> int:
        """Expert weight elements: w1 [E, 2I, H] plus w2 [E, H, I]."""
        return 3 * self.num_experts * self.intermediate * self.hidden

    def describe(self) -> str:
        e, h, i = self.num_experts, self.hidden, self.intermediate
        return f"E={e} H={h} I={i} (w1 [{e}, {2 * i}, {h}], w2 [{e}, {h}, {i}])"


def describe_fused_expert_block(module: nn.Module) -> Optional[ExpertBlockShape]:
    """The block's shape when ``module`` has the fused expert layout (unquantized or PACKED), else None."""
    pair = [getattr(module, name, None) for name in EXPERT_PARAM_NAMES]
    if not all(isinstance(t, torch.Tensor) and t.dim() == 3 for t in pair):
        return None
    held = is_packed_expert_block(module) or all(isinstance(t, nn.Parameter) for t in pair)
    (e1, rows1, h1), (e2, h2, i2) = (tuple(t.shape) for t in pair)
    if not held or e1 != e2 or h1 != h2 or rows1 != 2 * i2:
        return None
    return ExpertBlockShape(num_experts=e1, hidden=h1, intermediate=i2)


def is_fused_expert_block(module: nn.Module) -> bool:
    return describe_fused_expert_block(module) is not None


def _candidates(model: nn.Module, config: QuantConfig) -> Iterator[Tuple[str, nn.Module, ExpertBlockShape]]:
    for name, module in model.named_modules():
        shape = None if is_excluded(name, config) else describe_fused_expert_block(module)
        if shape is not None:
            yield name, module, shape


def find_expert_blocks(model: nn.Module, config: QuantConfig) -> List[Tuple[str, nn.Module, ExpertBlockShape]]:
    """Every non-excluded module with the fused expert layout, in module order."""
    return list(_candidates(model, config))


def _settle(block: nn.Module, weights: QuantExpertWeights, config: QuantConfig) -> None:
    """Attach the packed buffers and put ``block`` in the config's residency mode."""
    compute = getattr(torch, config.compute_dtype)
    attach_packed_buffers(block, weights, compute, config.compile_dequant)
    if config.mode is not ExecutionMode.PACKED:
        materialize_expert_params(block, weights, compute_dtype=compute)
    elif not is_packed_expert_block(block):
        install_packed_expert_access(block)


def _quantize_block(name: str, block: nn.Module, config: QuantConfig) -> TargetedModule:
    if is_packed_expert_block(block):
        raise RuntimeError(f"{name!r} is already quantized in PACKED mode")
    w1, w2 = (getattr(block, n) for n in EXPERT_PARAM_NAMES)
    source_bytes = sum(t.numel() * t.element_size() for t in (w1, w2))
    weights = QuantExpertWeights.quantize(
        w1.detach(), w2.detach(), bits=config.bits, group_size=config.group_size,
        scale_dtype=getattr(torch, config.scale_dtype), scale_search=config.scale_search,
        search_grid=config.search_grid,
    )
    _settle(block, weights, config)
    return TargetedModule(
        name=name,
        kind="expert",
        module_type=unpacked_class(type(block)).__name__,
        shapes={n: list(r.logical_shape) for n, r in zip(EXPERT_PARAM_NAMES, weights.results())},
        bits=config.bits,
        group_size=weights.w1.group_size,
        packed=weights.w1.packed,
        execution_mode=config.mode.value,
        source_bytes=source_bytes,
        quantized_bytes=weights.storage_bytes(),
    )


def quantize_llada_experts(model: nn.Module, config: QuantConfig) -> List[TargetedModule]:
    """Quantize every fused expert block in place in the config's residency mode; one record per block.

    The blocks are collected before any of them changes, so the walk never
    sees a half-converted model.
    """
    return [_quantize_block(name, block, config) for name, block, _ in find_expert_blocks(model, config)]


def restore_llada_experts_from_buffers(model: nn.Module, config: QuantConfig) -> int:
    """Re-wire every block holding the four packed buffers after a load; returns how many.

    PACKED: metadata re-attached and w1/w2 served from the buffers; REFERENCE:
    the BF16 Parameters rewritten from them.  The group length of each
    tensor comes from its scales, not from ``config``.
    """
    count = 0
    for block in model.modules():
        if any(getattr(block, n, None) is None for n in PACKED_BUFFERS):
            continue
        weights = QuantExpertWeights(
            quant_result_from_buffers(block._qw1, block._sw1, config.bits),
            quant_result_from_buffers(block._qw2, block._sw2, config.bits),
        )
        _settle(block, weights, config)
        count += 1
    return count
