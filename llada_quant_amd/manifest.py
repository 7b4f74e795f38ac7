"""Audit record of one quantized module (the ``TargetedModule`` of formats/manifest.py).

Only the record type is here: the on-disk checkpoint format of the reference
(``formats/``) is outside this package's scope.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field
from typing import Dict, List


@dataclass
class TargetedModule:
    """What quantization did to one module: name, kind, shapes, bits, bytes."""

    name: str
    kind: str
    module_type: str
    shapes: Dict[str, List[int]] = field(default_factory=dict)
    bits: int = 8
    group_size: int = 128
    packed: bool = False
    execution_mode: str = "packed"
    source_bytes: int = 0
    quantized_bytes: int = 0

    def to_dict(self) -> dict:
        return asdict(self)
