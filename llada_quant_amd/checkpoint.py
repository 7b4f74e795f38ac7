"""Packed checkpoints: save, and load straight into GPU buffers.

The on-disk layout is the reference's (formats/safetensors.py:1-15,
formats/manifest.py:60-110):

    <dir>/model-int{bits}.safetensors   packed codes + scales + untargeted tensors
    <dir>/quantization.json             manifest: config, targeted modules, totals

so checkpoints written by the reference load here and the other way round.
The BF16 expert weights ``w1``/``w2`` are never stored: the packed buffers
``_qw1/_sw1/_qw2/_sw2`` are the weights.  ``load_quantized_weights`` reads the
file with ``safetensors.torch.load_file(..., device=...)``, so the packed
buffers land in device memory without a host copy of the model; the expert
blocks are then re-wired to their packed buffers (adapters/llada_moe.py:163-186,
group sizes derived from the scales as runtime/moe.py:82-102 does).
"""

from __future__ import annotations

import glob
import json
import os
from dataclasses import asdict
from typing import List, Optional, Set, Tuple, Union

import torch
import torch.nn as nn
from safetensors.torch import load_file, save_file

from .config import FORMAT_VERSION, QuantConfig

MANIFEST_FILENAME = "quantization.json"
WEIGHTS_GLOB = "model-int*.safetensors"


def weights_filename(bits: int) -> str:
    return f"model-int{bits}.safetensors"


def derivable_tensor_names(manifest: dict) -> Set[str]:
    """The BF16 ``w1``/``w2`` of every expert target: re-derived from the packed buffers, never stored."""
    names: Set[str] = set()
    for target in manifest.get("targets", []):
        if target.get("kind") == "expert":
            prefix = f"{target['name']}." if target.get("name") else ""
            names.update({f"{prefix}w1", f"{prefix}w2"})
    return names


def _manifest(result) -> dict:
    """The reference's manifest dictionary (formats/manifest.py:93-108) for a QuantizationResult."""
    targets = [asdict(t) if not isinstance(t, dict) else t for t in result.targets]
    return {
        "format_version": FORMAT_VERSION,
        "framework_version": "llada_quant_amd",
        "created_at": "",
        "source_checkpoint": None,
        "config": result.config.to_dict(),
        "entries": [],
        "targets": targets,
        "totals": {
            "source_bytes": sum(t.get("source_bytes", 0) for t in targets),
            "quantized_bytes": sum(t.get("quantized_bytes", 0) for t in targets),
            "module_count": len(targets),
        },
    }


def save_quantized_checkpoint(model: nn.Module, result, directory: str) -> str:
    """Write the model's packed state and the manifest; returns the weights file path.

    ``result`` is the QuantizationResult of quantize_model (config + targets).
    """
    manifest = _manifest(result)
    os.makedirs(directory, exist_ok=True)
    path = os.path.join(directory, weights_filename(result.config.bits))
    skip = derivable_tensor_names(manifest)
    state = {name: t.detach().cpu().contiguous() for name, t in model.state_dict().items()
             if isinstance(t, torch.Tensor) and name not in skip}
    save_file(state, path)
    with open(os.path.join(directory, MANIFEST_FILENAME), "w") as f:
        json.dump(manifest, f, indent=2)
    return path


def find_weights_file(directory: str) -> str:
    matches = sorted(glob.glob(os.path.join(directory, WEIGHTS_GLOB)))
    if not matches:
        raise FileNotFoundError(f"no {WEIGHTS_GLOB} in {directory!r}")
    if len(matches) > 1:
        raise RuntimeError(f"ambiguous checkpoint, multiple weight files: {matches}")
    return matches[0]


def load_quantized_checkpoint(directory: str, device: Union[str, torch.device] = "cpu") -> Tuple[dict, dict]:
    """Packed tensors (placed on ``device`` by the safetensors reader) and the manifest dict."""
    with open(os.path.join(directory, MANIFEST_FILENAME)) as f:
        manifest = json.load(f)
    state = load_file(find_weights_file(directory), device=str(device))
    return state, manifest


def _register_missing_buffers(model: nn.Module, state: dict) -> List[str]:
    """Persistent buffers for checkpoint tensors the model lacks (a plain model absorbing packed experts)."""
    existing = set(model.state_dict().keys())
    registered: List[str] = []
    for name, tensor in state.items():
        if name in existing:
            continue
        parent_path, _, leaf = name.rpartition(".")
        try:
            module = model.get_submodule(parent_path) if parent_path else model
        except AttributeError as exc:
            raise RuntimeError(
                f"state dict mismatch: checkpoint holds {name!r} but the model has no submodule "
                f"{parent_path!r} ({exc}). The checkpoint was produced from a different architecture."
            ) from exc
        module.register_buffer(leaf, tensor, persistent=True)
        registered.append(name)
    return registered


def load_quantized_weights(model: nn.Module, directory: str, strict: bool = True,
                           device: Optional[Union[str, torch.device]] = None) -> dict:
    """Load a packed checkpoint into ``model`` (plain or already quantized); returns the manifest.

    With ``device`` (e.g. ``"cuda:0"``) the tensors are read straight into that
    device's memory and the model's matching tensors move there.  Missing
    packed buffers are registered; the BF16 expert weights are expected to be
    absent.  Any other missing or unexpected key raises when ``strict``.
    """
    state, manifest = load_quantized_checkpoint(directory, device if device is not None else "cpu")
    if device is not None:
        model.to(device)
    _register_missing_buffers(model, state)
    expected_missing = derivable_tensor_names(manifest)
    incompatible, unexpected = model.load_state_dict(state, strict=False)
    missing = [key for key in incompatible if key not in expected_missing]
    if strict and (missing or unexpected):
        raise RuntimeError(f"state dict mismatch: missing={missing}, unexpected={list(unexpected)}")
    if manifest.get("config"):
        from .adapters.llada_moe import restore_llada_experts_from_buffers

        restore_llada_experts_from_buffers(model, QuantConfig.from_dict(manifest["config"]))
    return manifest
