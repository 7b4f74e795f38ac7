"""Public API: quantize a model's fused expert blocks (api.py of the reference).

``quantize_model`` returns an audit trail and refuses to succeed quietly when
it matched nothing (api.py:102-135 of ``LLaDA_Quant`` v0.2.0).  Dense
``linear`` targets belong to the reference's QuantLinear path, which is not
part of this package: asking for them raises.
"""

from __future__ import annotations

import copy
from dataclasses import dataclass, field
from typing import List

import torch.nn as nn

from .adapters.llada_moe import quantize_llada_experts
from .config import COMPONENT_EXPERT, COMPONENT_LINEAR, ExecutionMode, QuantConfig
from .manifest import TargetedModule


class TargetingError(RuntimeError):
    """A run touched a different set of modules than intended."""


@dataclass
class QuantizationResult:
    config: QuantConfig
    targets: List[TargetedModule] = field(default_factory=list)

    @property
    def names(self) -> List[str]:
        return [t.name for t in self.targets]

    @property
    def expert_blocks(self) -> List[TargetedModule]:
        return [t for t in self.targets if t.kind == "expert"]

    @property
    def linears(self) -> List[TargetedModule]:
        return [t for t in self.targets if t.kind == "linear"]

    @property
    def source_bytes(self) -> int:
        return sum(t.source_bytes for t in self.targets)

    @property
    def quantized_bytes(self) -> int:
        return sum(t.quantized_bytes for t in self.targets)

    @property
    def weight_ratio(self) -> float:
        return self.quantized_bytes / self.source_bytes if self.source_bytes else 1.0

    def summary(self) -> str:
        mode = self.config.mode
        lines = [
            f"quantized {len(self.targets)} module(s): "
            f"{len(self.expert_blocks)} expert block(s), {len(self.linears)} linear(s)",
            f"bits={self.config.bits} group_size={self.config.group_size} "
            f"mode={mode.value} packed={any(t.packed for t in self.targets)}",
            f"converted weights: {self.source_bytes / 2**20:.2f} MiB -> "
            f"{self.quantized_bytes / 2**20:.2f} MiB ({self.weight_ratio:.3f}x)",
        ]
        if mode is ExecutionMode.REFERENCE:
            lines.append("REFERENCE mode: dequantized BF16 weights are still resident next to "
                         "the packed ones. The model is LARGER than unquantized. Validation only.")
        else:
            lines.append("PACKED mode: only codes and scales are resident; fused_moe consumes "
                         "them directly on the GPU.")
        return "\n".join(lines)


def _validate_targeting(result: QuantizationResult, config: QuantConfig) -> None:
    if not result.targets and not config.allow_no_matches:
        raise TargetingError(
            f"quantization matched no modules for targets={list(config.targets)}. "
            "A silent no-op is indistinguishable from success, so this is an error. "
            "For experts, check the block really has w1 [E, 2I, H] / w2 [E, H, I] "
            "Parameters. Pass allow_no_matches=True only in tests."
        )
    if config.expect_expert_blocks is not None and len(result.expert_blocks) != config.expect_expert_blocks:
        raise TargetingError(
            f"expected {config.expect_expert_blocks} expert block(s), matched {len(result.expert_blocks)}: "
            f"{[t.name for t in result.expert_blocks]}"
        )
    if config.expect_linears is not None and len(result.linears) != config.expect_linears:
        raise TargetingError(
            f"expected {config.expect_linears} linear(s), matched {len(result.linears)}: "
            f"{[t.name for t in result.linears]}"
        )


def quantize_model(model: nn.Module, config: QuantConfig) -> QuantizationResult:
    """Quantize every fused expert block of ``model`` in place (on its GPU)."""
    if COMPONENT_LINEAR in config.targets:
        raise NotImplementedError(
            "dense linear targets (QuantLinear) are not part of the packed expert path; "
            "use targets=('expert',)"
        )
    targets: List[TargetedModule] = []
    if COMPONENT_EXPERT in config.targets:
        targets += quantize_llada_experts(model, config)
    result = QuantizationResult(config=config, targets=targets)
    _validate_targeting(result, config)
    return result


def quantized_model(model: nn.Module, config: QuantConfig) -> nn.Module:
    """A quantized deep copy of ``model``."""
    clone = copy.deepcopy(model)
    quantize_model(clone, config)
    return clone
