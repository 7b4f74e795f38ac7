"""LLaDA-MoE adapter: structural detection of fused expert blocks, quantize, restore.

Drop-in for ``LLaDA_Quant.adapters.llada_moe`` (v0.2.0,
``src/LLaDA_Quant/adapters/llada_moe.py``).  A module is a fused expert
block when its ``w1``/``w2`` have the layout of ``TritonFusedMoEBlock``::

    w1 [E, 2I, H] and w2 [E, H, I]:  same E, same H, w1 rows = 2 * w2 cols

Detection is structural, never by name.  Quantization runs on the GPU (the
block's weights must be on a ROCm device) through the HIP quantizer.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
import torch.nn as nn

from ..config import ExecutionMode, QuantConfig, is_excluded
from ..manifest import TargetedModule
from ..runtime.moe import (
    PACKED_BUFFERS,
    QuantExpertWeights,
    attach_packed_buffers,
    install_packed_expert_access,
    is_packed_expert_block,
    materialize_expert_params,
    quant_result_from_buffers,
)


@dataclass(frozen=True)
class ExpertBlockShape:
    """The numbers that identify a fused expert block (llada_moe.py:43-61)."""

    num_experts: int
    hidden: int
    intermediate: int

    @property
    def numel(self) -> int:
        """Expert weight elements: w1 [E, 2I, H] plus w2 [E, H, I]."""
        return self.num_experts * 3 * self.intermediate * self.hidden

    def describe(self) -> str:
        e, h, i = self.num_experts, self.hidden, self.intermediate
        return f"E={e} H={h} I={i} (w1 [{e}, {2 * i}, {h}], w2 [{e}, {h}, {i}])"


def describe_fused_expert_block(module: nn.Module) -> Optional[ExpertBlockShape]:
    """The block's shape if it is a fused expert block (BF16 or PACKED), else None."""
    w1 = getattr(module, "w1", None)
    w2 = getattr(module, "w2", None)
    if not isinstance(w1, torch.Tensor) or not isinstance(w2, torch.Tensor):
        return None
    if not is_packed_expert_block(module) and not (isinstance(w1, nn.Parameter) and isinstance(w2, nn.Parameter)):
        return None
    if w1.dim() != 3 or w2.dim() != 3:
        return None
    experts, two_i, hidden = w1.shape
    experts2, hidden2, intermediate = w2.shape
    if experts != experts2 or hidden != hidden2 or two_i != 2 * intermediate:
        return None
    return ExpertBlockShape(num_experts=experts, hidden=hidden, intermediate=intermediate)


def is_fused_expert_block(module: nn.Module) -> bool:
    return describe_fused_expert_block(module) is not None


def find_expert_blocks(model: nn.Module, config: QuantConfig) -> List[Tuple[str, nn.Module, ExpertBlockShape]]:
    """Every structurally matching, non-excluded fused expert block."""
    found = []
    for name, block in model.named_modules():
        if is_excluded(name, config):
            continue
        shape = describe_fused_expert_block(block)
        if shape is not None:
            found.append((name, block, shape))
    return found


def quantize_llada_experts(model: nn.Module, config: QuantConfig) -> List[TargetedModule]:
    """Quantize every fused expert block in place (llada_moe.py:108-160)."""
    compute_dtype = getattr(torch, config.compute_dtype)
    scale_dtype = getattr(torch, config.scale_dtype)
    mode = config.mode
    records: List[TargetedModule] = []
    for name, block, _shape in find_expert_blocks(model, config):
        if is_packed_expert_block(block):
            raise RuntimeError(f"{name!r} is already quantized in PACKED mode")
        bf16_bytes = sum(p.numel() * p.element_size() for p in (block.w1, block.w2))
        weights = QuantExpertWeights.quantize(
            block.w1.detach(), block.w2.detach(), bits=config.bits, group_size=config.group_size,
            scale_dtype=scale_dtype, scale_search=config.scale_search, search_grid=config.search_grid,
        )
        attach_packed_buffers(block, weights, compute_dtype, config.compile_dequant)
        if mode is ExecutionMode.PACKED:
            install_packed_expert_access(block)
        else:
            materialize_expert_params(block, weights, compute_dtype=compute_dtype)
        records.append(TargetedModule(
            name=name,
            kind="expert",
            module_type=type(block).__mro__[1].__name__ if mode is ExecutionMode.PACKED else type(block).__name__,
            shapes={"w1": list(weights.w1.logical_shape), "w2": list(weights.w2.logical_shape)},
            bits=config.bits,
            group_size=weights.w1.group_size,
            packed=weights.w1.packed,
            execution_mode=mode.value,
            source_bytes=bf16_bytes,
            quantized_bytes=weights.storage_bytes(),
        ))
    return records


def restore_llada_experts_from_buffers(model: nn.Module, config: QuantConfig) -> int:
    """Re-establish expert weight access after a bare buffer load (llada_moe.py:163-186)."""
    compute_dtype = getattr(torch, config.compute_dtype)
    touched = 0
    for block in model.modules():
        if not all(hasattr(block, b) for b in PACKED_BUFFERS):
            continue
        weights = QuantExpertWeights(
            w1=quant_result_from_buffers(block._qw1, block._sw1, config.bits),
            w2=quant_result_from_buffers(block._qw2, block._sw2, config.bits),
        )
        attach_packed_buffers(block, weights, compute_dtype, config.compile_dequant)
        if config.mode is ExecutionMode.PACKED:
            if not is_packed_expert_block(block):
                install_packed_expert_access(block)
        else:
            materialize_expert_params(block, weights, compute_dtype=compute_dtype)
        touched += 1
    return touched
