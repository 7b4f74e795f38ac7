"""Manifest of a quantized checkpoint: what produced it and what it converted.

The JSON written here is the reference's ``quantization.json`` key for key
(``formats/manifest.py:60-129`` of LLaDA_Quant v0.2.0), so a manifest written
by either framework reads in the other: ``format_version``,
``framework_version``, ``created_at``, ``source_checkpoint``, ``config``
(``QuantConfig.to_dict``), ``entries`` (per tensor), ``targets`` (per
converted module, with measured byte counts) and ``totals``.  The source
pointer goes to ``source-checkpoint.json`` (``:138-144``).
"""

from __future__ import annotations

import dataclasses
import hashlib
import json
import os
from dataclasses import dataclass, field
from datetime import datetime, timezone
from typing import Dict, List, Optional

import torch

from ..config import FORMAT_VERSION, QuantConfig

MANIFEST_FILENAME = "quantization.json"
SOURCE_FILENAME = "source-checkpoint.json"
FRAMEWORK_VERSION = "llada_quant_amd 0.2"


@dataclass
class TargetedModule:
    """One converted module: its name and kind, shapes, format and measured bytes."""

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

    @property
    def compression_ratio(self) -> float:
        """quantized / source bytes (1.0 when nothing was measured)."""
        return self.quantized_bytes / self.source_bytes if self.source_bytes else 1.0

    def to_dict(self) -> dict:
        return dataclasses.asdict(self)


@dataclass
class QuantEntry:
    """One stored quantized tensor."""

    tensor_name: str
    shape: List[int]
    bits: int
    group_size: int
    storage_dtype: str
    compute_dtype: str
    source_tensor: Optional[str] = None
    sha256: Optional[str] = None


def _record(cls, data: dict):
    """A dataclass record from a JSON object; keys the record does not know are ignored."""
    names = {f.name for f in dataclasses.fields(cls)}
    return cls(**{k: v for k, v in data.items() if k in names})


def _utc_now() -> str:
    return datetime.now(timezone.utc).isoformat()


@dataclass
class QuantizationManifest:
    """Everything that produced one checkpoint."""

    format_version: int = FORMAT_VERSION
    framework_version: str = FRAMEWORK_VERSION
    created_at: str = field(default_factory=_utc_now)
    source_checkpoint: Optional[str] = None
    config: Optional[QuantConfig] = None
    entries: List[QuantEntry] = field(default_factory=list)
    targets: List[TargetedModule] = field(default_factory=list)

    @property
    def source_bytes(self) -> int:
        return sum(t.source_bytes for t in self.targets)

    @property
    def quantized_bytes(self) -> int:
        return sum(t.quantized_bytes for t in self.targets)

    def to_dict(self) -> dict:
        out = {
            "format_version": self.format_version,
            "framework_version": self.framework_version,
            "created_at": self.created_at,
            "source_checkpoint": self.source_checkpoint,
            "config": None if self.config is None else self.config.to_dict(),
            "entries": [dataclasses.asdict(e) for e in self.entries],
            "targets": [dataclasses.asdict(t) for t in self.targets],
        }
        out["totals"] = {"source_bytes": self.source_bytes, "quantized_bytes": self.quantized_bytes,
                         "module_count": len(self.targets)}
        return out

    @classmethod
    def from_dict(cls, data: dict) -> "QuantizationManifest":
        cfg = data.get("config")
        return cls(
            format_version=data.get("format_version", FORMAT_VERSION),
            framework_version=data.get("framework_version", "unknown"),
            created_at=data.get("created_at", ""),
            source_checkpoint=data.get("source_checkpoint"),
            config=QuantConfig.from_dict(cfg) if cfg else None,
            entries=[_record(QuantEntry, e) for e in data.get("entries", [])],
            targets=[_record(TargetedModule, t) for t in data.get("targets", [])],
        )

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), indent=2, sort_keys=True)

    def save(self, directory: str) -> None:
        """Write ``quantization.json`` into ``directory``."""
        with open(os.path.join(directory, MANIFEST_FILENAME), "w") as f:
            f.write(self.to_json())

    @classmethod
    def load(cls, directory: str) -> "QuantizationManifest":
        with open(os.path.join(directory, MANIFEST_FILENAME)) as f:
            return cls.from_dict(json.load(f))


def _file_sha256(path: str) -> str:
    digest = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            block = f.read(1 << 20)
            if not block:
                return digest.hexdigest()
            digest.update(block)


def tensor_hash(t: torch.Tensor) -> str:
    """SHA-256 of a tensor's values as contiguous float32 on the host."""
    values = t.detach().to(device="cpu", dtype=torch.float32).contiguous()
    return hashlib.sha256(values.numpy().tobytes()).hexdigest()


def write_source_checkpoint_meta(directory: str, source: Optional[str]) -> None:
    """``source-checkpoint.json``: the unquantized source, with its SHA-256 when it is a local file."""
    meta: Dict[str, Optional[str]] = {"source_checkpoint": source}
    if source is not None and os.path.isfile(source):
        meta["source_sha256"] = _file_sha256(source)
    with open(os.path.join(directory, SOURCE_FILENAME), "w") as f:
        json.dump(meta, f, indent=2, sort_keys=True)
