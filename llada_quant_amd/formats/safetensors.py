"""The quantized artifact: ``model-int{bits}.safetensors`` + manifest, and loading it onto a GPU.

Directory layout (the reference's, ``formats/safetensors.py:1-15`` of
LLaDA_Quant v0.2.0, so artifacts move between the two frameworks)::

    model-int{bits}.safetensors   packed codes and scales, every untargeted tensor
    quantization.json             the manifest (formats/manifest.py)
    source-checkpoint.json        the unquantized source it came from

The BF16 ``w1``/``w2`` of an expert block are never written: the packed
buffers ``_qw1/_sw1/_qw2/_sw2`` are the weights, and a model loading the
artifact derives ``w1``/``w2`` from them again.  Loading reads the tensors
straight into the memory of ``device`` (``safetensors.torch.load_file``), so a
checkpoint goes to HBM without a host copy of the model; buffers the model
lacks (a plain model absorbing packed experts) are registered as they arrive.
"""

from __future__ import annotations

import glob
import os
from typing import Dict, Optional, Set, Tuple, Union

import torch
import torch.nn as nn
from safetensors.torch import load_file, save_file

from .manifest import QuantizationManifest, TargetedModule, _record, write_source_checkpoint_meta

WEIGHTS_GLOB = "model-int*.safetensors"

Device = Union[str, torch.device]


def weights_filename(bits: int) -> str:
    return f"model-int{bits}.safetensors"


def _targets(manifest) -> list:
    if isinstance(manifest, QuantizationManifest):
        return manifest.targets
    return [_record(TargetedModule, t) for t in manifest.get("targets", [])]


def derivable_tensor_names(manifest) -> Set[str]:
    """State-dict names an artifact leaves out because the packed buffers rebuild them:
    ``<block>.w1`` and ``<block>.w2`` of every expert target (manifest object or its JSON dict)."""
    names: Set[str] = set()
    for t in _targets(manifest):
        if t.kind == "expert":
            names.update(f"{t.name}.{w}" if t.name else w for w in ("w1", "w2"))
    return names


def collect_quantized_state(model: nn.Module, manifest=None) -> Dict[str, torch.Tensor]:
    """Host copies of the model's state without the derivable BF16 expert weights."""
    skip = derivable_tensor_names(manifest) if manifest is not None else set()
    state = {}
    for name, t in model.state_dict().items():
        if isinstance(t, torch.Tensor) and name not in skip:
            state[name] = t.detach().to("cpu").contiguous()
    return state


def _as_manifest(manifest) -> QuantizationManifest:
    """A QuantizationManifest as is; anything carrying ``config`` and ``targets``
    (a QuantizationResult) becomes one."""
    if isinstance(manifest, QuantizationManifest):
        return manifest
    return QuantizationManifest(config=manifest.config, targets=list(manifest.targets),
                                source_checkpoint=getattr(manifest.config, "source_checkpoint", None))


def save_quantized_checkpoint(model: nn.Module, manifest, directory: str, weights_file: Optional[str] = None) -> str:
    """Write the artifact into ``directory``; returns the weights file's path."""
    manifest = _as_manifest(manifest)
    os.makedirs(directory, exist_ok=True)
    bits = manifest.config.bits if manifest.config is not None else 8
    path = os.path.join(directory, weights_file or weights_filename(bits))
    save_file(collect_quantized_state(model, manifest), path)
    manifest.save(directory)
    write_source_checkpoint_meta(directory, manifest.source_checkpoint)
    return path


def find_weights_file(directory: str) -> str:
    """The one ``model-int*.safetensors`` of an artifact directory."""
    found = sorted(glob.glob(os.path.join(directory, WEIGHTS_GLOB)))
    if not found:
        raise FileNotFoundError(f"no {WEIGHTS_GLOB} in {directory!r}")
    if len(found) > 1:
        raise RuntimeError(f"ambiguous checkpoint, multiple weight files: {found}")
    return found[0]


def checkpoint_size_bytes(directory: str) -> int:
    """Bytes on disk of every file of the artifact."""
    total = 0
    for entry in os.scandir(directory):
        if entry.is_file():
            total += entry.stat().st_size
    return total


def load_quantized_checkpoint(directory: str, device: Device = "cpu") -> Tuple[Dict[str, torch.Tensor],
                                                                                QuantizationManifest]:
    """The artifact's tensors (in ``device`` memory) and its manifest; no model is touched."""
    manifest = QuantizationManifest.load(directory)
    return load_file(find_weights_file(directory), device=str(device)), manifest


def load_quantized_weights(model: nn.Module, directory: str, strict: bool = True,
                           device: Optional[Device] = None) -> QuantizationManifest:
    """Load an artifact into ``model`` (plain or already quantized); returns its manifest.

    With ``device`` (e.g. ``"cuda:0"``) the tensors are read into that
    device's memory and the model moves there first.  Checkpoint tensors
    the model has no slot for become persistent buffers of their owning
    module; a tensor whose owning module does not exist means another
    architecture and raises.  The BF16 expert weights are expected to be
    absent; any other missing or unexpected key raises when ``strict``.
    The expert blocks are then re-wired to their packed buffers under the
    manifest's config (PACKED: served from the buffers; REFERENCE: BF16
    Parameters rewritten by the dequant kernel).
    """
    state, manifest = load_quantized_checkpoint(directory, device if device is not None else "cpu")
    if device is not None:
        model.to(device)
    modules = dict(model.named_modules())
    present = set(model.state_dict().keys())
    adopted = set()
    for key, tensor in state.items():
        if key in present:
            continue
        owner, _, leaf = key.rpartition(".")
        module = modules.get(owner)
        if module is None:
            raise RuntimeError(
                f"state dict mismatch: checkpoint holds {key!r} but the model has no submodule {owner!r}; "
                "the checkpoint was produced from a different architecture"
            )
        module.register_buffer(leaf, tensor, persistent=True)
        adopted.add(key)
    result = model.load_state_dict({k: v for k, v in state.items() if k not in adopted}, strict=False)
    missing = sorted(set(result.missing_keys) - adopted - derivable_tensor_names(manifest))
    if strict and (missing or result.unexpected_keys):
        raise RuntimeError(f"state dict mismatch: missing={missing}, unexpected={list(result.unexpected_keys)}")
    if manifest.config is not None:
        from ..adapters.llada_moe import restore_llada_experts_from_buffers

        restore_llada_experts_from_buffers(model, manifest.config)
    return manifest
