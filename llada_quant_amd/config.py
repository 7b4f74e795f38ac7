"""Quantization configuration and target selection.

Drop-in for ``LLaDA_Quant.config`` (v0.2.0, ``src/LLaDA_Quant/config.py``):
``ExecutionMode`` (``:32-51``), the frozen ``QuantConfig`` with its validation
and dict/JSON round trip (``:59-127``) and the glob-based exclusion policy
(``:29``, ``:130-144``).
"""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass
from enum import Enum
from fnmatch import fnmatch
from typing import Optional, Tuple

FORMAT_VERSION = 2

#: Module-path components never quantized (fnmatch globs per dotted part).
DEFAULT_EXCLUDES = ("router", "gate", "*norm*", "embed_tokens", "lm_head")


class ExecutionMode(str, Enum):
    """What stays resident after quantization.

    ``REFERENCE`` keeps dequantized BF16 Parameters next to the packed buffers
    (validation only; larger than the unquantized model).  ``PACKED`` keeps
    only codes and scales; ``block.w1``/``block.w2`` are served from them and
    :func:`llada_quant_amd.fused_moe` consumes them without dequantizing to HBM.
    """

    REFERENCE = "reference"
    PACKED = "packed"


COMPONENT_LINEAR = "linear"
COMPONENT_EXPERT = "expert"
KNOWN_TARGETS = (COMPONENT_EXPERT, COMPONENT_LINEAR)


@dataclass(frozen=True)
class QuantConfig:
    bits: int = 8
    group_size: int = 128
    targets: Tuple[str, ...] = (COMPONENT_EXPERT,)
    execution_mode: str = ExecutionMode.PACKED.value
    linear_include: Tuple[str, ...] = ()
    exclude: Tuple[str, ...] = DEFAULT_EXCLUDES
    compute_dtype: str = "bfloat16"
    scale_dtype: str = "float32"
    scale_search: str = "amax"
    search_grid: int = 24
    compile_dequant: bool = False
    source_checkpoint: Optional[str] = None
    expect_expert_blocks: Optional[int] = None
    expect_linears: Optional[int] = None
    allow_no_matches: bool = False

    def __post_init__(self) -> None:
        if self.bits not in (8, 4):
            raise ValueError(f"bits must be 8 or 4, got {self.bits}")
        if self.group_size <= 0 and self.group_size != -1:
            raise ValueError(f"group_size must be > 0 or -1, got {self.group_size}")
        if self.bits == 4 and self.group_size != -1 and self.group_size % 2 != 0:
            raise ValueError(
                f"bits=4 needs an even group_size so int4 groups stay byte-aligned, got {self.group_size}"
            )
        if self.scale_search not in ("amax", "mse"):
            raise ValueError(f"scale_search must be 'amax' or 'mse', got {self.scale_search!r}")
        if self.search_grid < 1:
            raise ValueError(f"search_grid must be >= 1, got {self.search_grid}")
        unknown = [t for t in self.targets if t not in KNOWN_TARGETS]
        if unknown:
            raise ValueError(f"unknown targets {unknown}; known: {list(KNOWN_TARGETS)}")
        try:
            ExecutionMode(self.execution_mode)
        except ValueError:
            raise ValueError(
                f"execution_mode must be one of {[m.value for m in ExecutionMode]}, got {self.execution_mode!r}"
            ) from None

    @property
    def mode(self) -> ExecutionMode:
        return ExecutionMode(self.execution_mode)

    @property
    def reduces_memory(self) -> bool:
        return self.mode is ExecutionMode.PACKED

    def to_dict(self) -> dict:
        return {"format_version": FORMAT_VERSION, **asdict(self)}

    @classmethod
    def from_dict(cls, data: dict) -> "QuantConfig":
        data = dict(data)
        for key in ("targets", "exclude", "linear_include"):
            if key in data and isinstance(data[key], list):
                data[key] = tuple(data[key])
        known = set(cls.__dataclass_fields__)
        return cls(**{k: v for k, v in data.items() if k in known})

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), indent=2, sort_keys=True)


def is_excluded(module_name: str, config: QuantConfig) -> bool:
    """True when any dotted component of ``module_name`` matches an exclude glob."""
    return any(fnmatch(part, pattern) for part in module_name.split(".") for pattern in config.exclude)


def matches_linear(module_name: str, config: QuantConfig) -> bool:
    """True when a dense linear is explicitly targeted (config.py:135-144)."""
    if COMPONENT_LINEAR not in config.targets or not config.linear_include:
        return False
    if is_excluded(module_name, config):
        return False
    leaf = module_name.rsplit(".", 1)[-1]
    return any(fnmatch(leaf, p) or fnmatch(module_name, p) for p in config.linear_include)
