"""Public API: quantize a model's fused expert blocks, with an audit trail.

Drop-in for the expert half of ``LLaDA_Quant.api`` (v0.2.0): ``quantize_model``
returns a :class:`QuantizationResult` naming every module it converted and
raises :class:`TargetingError` when the run touched a different set of modules
than the config expects, including none at all.  Dense ``linear`` targets
belong to the reference's ``adapters/torch.py`` (module replacement), which is
not part of this package: asking for them raises.

Typical use::

    config = QuantConfig(bits=4, group_size=128, scale_search="mse", expect_expert_blocks=16)
    result = quantize_model(model, config)          # on the GPU holding the model
    save_quantized_checkpoint(model, QuantizationManifest(config=config, targets=result.targets), "out")
"""

from __future__ import annotations

import copy
from dataclasses import dataclass, field
from typing import List, Optional

import torch.nn as nn

from .adapters.llada_moe import quantize_llada_experts
from .config import COMPONENT_EXPERT, COMPONENT_LINEAR, ExecutionMode, QuantConfig
from .formats.manifest import QuantizationManifest, TargetedModule
from .formats.safetensors import load_quantized_weights, save_quantized_checkpoint

__all__ = [
    "QuantConfig",
    "QuantizationManifest",
    "QuantizationResult",
    "TargetingError",
    "quantize_model",
    "quantized_model",
    "save_quantized_checkpoint",
    "load_quantized_weights",
]


class TargetingError(RuntimeError):
    """A run touched a different set of modules than the config asked for."""


_MIB = float(1 << 20)


@dataclass
class QuantizationResult:
    """What one ``quantize_model`` call converted."""

    config: QuantConfig
    targets: List[TargetedModule] = field(default_factory=list)

    def _of_kind(self, kind: str) -> List[TargetedModule]:
        return [t for t in self.targets if t.kind == kind]

    @property
    def names(self) -> List[str]:
        return [t.name for t in self.targets]

    @property
    def expert_blocks(self) -> List[TargetedModule]:
        return self._of_kind("expert")

    @property
    def linears(self) -> List[TargetedModule]:
        return self._of_kind("linear")

    @property
    def source_bytes(self) -> int:
        return sum(t.source_bytes for t in self.targets)

    @property
    def quantized_bytes(self) -> int:
        return sum(t.quantized_bytes for t in self.targets)

    @property
    def weight_ratio(self) -> float:
        src = self.source_bytes
        return self.quantized_bytes / src if src else 1.0

    def manifest(self, source_checkpoint: Optional[str] = None) -> QuantizationManifest:
        """The checkpoint manifest of this run."""
        return QuantizationManifest(config=self.config, targets=list(self.targets),
                                    source_checkpoint=source_checkpoint or self.config.source_checkpoint)

    def summary(self) -> str:
        cfg = self.config
        packed = any(t.packed for t in self.targets)
        text = [
            f"quantized {len(self.targets)} module(s): {len(self.expert_blocks)} expert block(s), "
            f"{len(self.linears)} linear(s)",
            f"bits={cfg.bits} group_size={cfg.group_size} mode={cfg.mode.value} packed={packed}",
            f"converted weights: {self.source_bytes / _MIB:.2f} MiB -> {self.quantized_bytes / _MIB:.2f} MiB "
            f"({self.weight_ratio:.3f}x)",
        ]
        if cfg.mode is ExecutionMode.REFERENCE:
            text.append("REFERENCE mode: the dequantized BF16 weights stay resident beside the codes, so the "
                        "model is LARGER than unquantized. Validation only.")
        else:
            text.append("PACKED mode: only codes and scales are resident, so Resident memory drops to the "
                        "packed size; fused_moe reads the codes on the GPU and block.w1 / block.w2 dequantize "
                        "on access.")
        return "\n".join(text)


def _check_targets(result: QuantizationResult, config: QuantConfig) -> None:
    """Raise TargetingError unless the run matched what the config expects."""
    if not result.targets and not config.allow_no_matches:
        raise TargetingError(
            f"quantization matched no modules for targets={list(config.targets)}. A silent no-op is "
            "indistinguishable from success, so this is an error. For experts, check the block really has "
            "w1 [E, 2I, H] / w2 [E, H, I] Parameters. Pass allow_no_matches=True only in tests."
        )
    for kind, want, got in (("expert block", config.expect_expert_blocks, result.expert_blocks),
                            ("linear", config.expect_linears, result.linears)):
        if want is not None and len(got) != want:
            raise TargetingError(f"expected {want} {kind}(s), matched {len(got)}: {[t.name for t in got]}")


def quantize_model(model: nn.Module, config: QuantConfig) -> QuantizationResult:
    """Quantize every fused expert block of ``model`` in place, on the GPU holding its weights."""
    if COMPONENT_LINEAR in config.targets:
        raise NotImplementedError(
            "dense linear targets (QuantLinear module replacement) are not part of the packed expert path; "
            "use targets=('expert',), or QuantLinear.from_linear for a single layer"
        )
    found = quantize_llada_experts(model, config) if COMPONENT_EXPERT in config.targets else []
    result = QuantizationResult(config=config, targets=found)
    _check_targets(result, config)
    return result


def quantized_model(model: nn.Module, config: QuantConfig) -> nn.Module:
    """A quantized deep copy of ``model``; ``model`` itself is left as it was."""
    clone = copy.deepcopy(model)
    quantize_model(clone, config)
    return clone
