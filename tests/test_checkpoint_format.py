"""The checkpoint format without a GPU, against artifacts the reference itself wrote.

``tests/golden/ckpt_*`` were produced by LLaDA_Quant v0.2.0's own
``quantize_model`` + ``save_quantized_checkpoint`` on its test model
(tests/golden/make_ckpt_golden.py; the cases of
tests/unit/test_checkpoint_format.py:115-175).  Here they are read by this
package: the manifest parses to the same config and targets, a plain model on
the host absorbs the packed buffers in PACKED mode (no dequantization needed,
so no GPU), a model of another architecture is refused, and saving the loaded
model again reproduces the reference's tensors and manifest keys.  The GPU
side (``block.w1`` bits, REFERENCE mode) is tests/test_gpu_checkpoint.py.
"""

from __future__ import annotations

import json
import os

import pytest
import torch
from safetensors.torch import load_file

from conftest import ToyMoE
from llada_quant_amd import ExecutionMode, QuantConfig, QuantizationManifest, load_quantized_weights
from llada_quant_amd.formats.manifest import (
    MANIFEST_FILENAME,
    SOURCE_FILENAME,
    QuantEntry,
    TargetedModule,
    tensor_hash,
)
from llada_quant_amd.formats.safetensors import (
    checkpoint_size_bytes,
    derivable_tensor_names,
    find_weights_file,
    load_quantized_checkpoint,
    save_quantized_checkpoint,
    weights_filename,
)
from llada_quant_amd.runtime.moe import PACKED_BUFFERS, PackedExpertTensor, is_packed_expert_block

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = {"int4_packed_g64": (4, 64, "packed"), "int8_reference_g64": (8, 64, "reference"),
         "int8_packed_g48": (8, 48, "packed")}


def ref_dir(case):
    return os.path.join(GOLDEN, f"ckpt_{case}")


@pytest.mark.parametrize("case", sorted(CASES))
def test_reference_manifest_parses(case):
    bits, group, mode = CASES[case]
    manifest = QuantizationManifest.load(ref_dir(case))
    assert manifest.config == QuantConfig(bits=bits, group_size=group, targets=("expert",), execution_mode=mode)
    assert manifest.framework_version == "0.2.0" and manifest.source_checkpoint == "hf://test/model"
    assert [t.name for t in manifest.targets] == ["layers.0.mlp", "layers.1.mlp"]
    assert all(t.kind == "expert" and t.bits == bits and t.packed == (bits == 4) for t in manifest.targets)
    # the reference records the group length the quantizer used (-1: the per-row fallback)
    assert all(t.group_size == (group if 128 % group == 0 else -1) for t in manifest.targets)
    raw = json.load(open(os.path.join(ref_dir(case), MANIFEST_FILENAME)))
    assert manifest.to_dict()["totals"] == raw["totals"]
    assert derivable_tensor_names(manifest) == derivable_tensor_names(raw) == {
        "layers.0.mlp.w1", "layers.0.mlp.w2", "layers.1.mlp.w1", "layers.1.mlp.w2"}


def test_manifest_json_has_the_reference_layout():
    """Every key the reference writes, at every level, and nothing else."""
    raw = json.load(open(os.path.join(ref_dir("int4_packed_g64"), MANIFEST_FILENAME)))
    mine = json.loads(QuantizationManifest.from_dict(raw).to_json())
    assert set(mine) == set(raw)
    assert set(mine["config"]) == set(raw["config"])
    assert set(mine["targets"][0]) == set(raw["targets"][0])
    for key in ("config", "targets", "totals", "source_checkpoint", "format_version", "created_at"):
        assert mine[key] == raw[key], key


def test_manifest_round_trip_and_records():
    config = QuantConfig(bits=4, group_size=64)
    manifest = QuantizationManifest(
        source_checkpoint="hf://x", config=config,
        entries=[QuantEntry("w1", [1, 2], 4, 64, "int8", "bfloat16")],
        targets=[TargetedModule("m", "expert", "B", {"w1": [1, 2]}, 4, 64, True, "packed", 8, 3)],
    )
    back = QuantizationManifest.from_dict(json.loads(manifest.to_json()))
    assert back.config == config and back.entries == manifest.entries and back.targets == manifest.targets
    assert back.targets[0].packed is True and back.targets[0].compression_ratio == 3 / 8
    # unknown keys in a record are ignored (a newer writer), missing optional ones take defaults
    t = QuantizationManifest.from_dict({"targets": [{"name": "a", "kind": "expert", "module_type": "B",
                                                     "future_field": 1}]}).targets[0]
    assert t.name == "a" and t.bits == 8


def test_derivable_names_lists_only_expert_weights():
    manifest = QuantizationManifest(targets=[
        TargetedModule("layers.0.mlp", "expert", "Block", {}, 8, 64, False, "packed", 10, 5),
        TargetedModule("layers.0.q_proj", "linear", "Linear", {}, 8, 64, False, "packed", 4, 2),
        TargetedModule("", "expert", "Block", {}, 8, 64, False, "packed", 4, 2),
    ])
    assert derivable_tensor_names(manifest) == {"layers.0.mlp.w1", "layers.0.mlp.w2", "w1", "w2"}


def test_weights_file_lookup_and_size(tmp_path):
    assert weights_filename(4) == "model-int4.safetensors"
    with pytest.raises(FileNotFoundError):
        find_weights_file(str(tmp_path))
    (tmp_path / "model-int4.safetensors").write_bytes(b"x" * 10)
    (tmp_path / "quantization.json").write_bytes(b"{}")
    assert find_weights_file(str(tmp_path)).endswith("model-int4.safetensors")
    assert checkpoint_size_bytes(str(tmp_path)) == 12
    (tmp_path / "model-int8.safetensors").write_bytes(b"")
    with pytest.raises(RuntimeError, match="ambiguous"):
        find_weights_file(str(tmp_path))


def test_tensor_hash_is_value_deterministic():
    a = torch.arange(6, dtype=torch.float32).reshape(2, 3)
    assert tensor_hash(a) == tensor_hash(a.clone()) == tensor_hash(a.to(torch.float64))
    assert tensor_hash(a) != tensor_hash(a + 1)


@pytest.mark.parametrize("case", ["int4_packed_g64", "int8_packed_g48"])
def test_plain_host_model_absorbs_a_reference_packed_checkpoint(case):
    bits = CASES[case][0]
    model = ToyMoE(seed=123)  # different BF16 weights; w1/w2 are Parameters until the load
    manifest = load_quantized_weights(model, ref_dir(case))
    assert isinstance(manifest, QuantizationManifest) and manifest.config.mode is ExecutionMode.PACKED
    stored = load_file(find_weights_file(ref_dir(case)))
    for i, layer in enumerate(model.layers):
        block = layer.mlp
        assert is_packed_expert_block(block)
        assert "w1" not in dict(block.named_parameters())
        for name in PACKED_BUFFERS:
            assert torch.equal(getattr(block, name), stored[f"layers.{i}.mlp.{name}"])
        assert isinstance(block.w1, PackedExpertTensor) and block.w1.shape == (4, 128, 128)
        assert block.w1.bits == bits and block.w2.shape == (4, 128, 64)
        assert torch.equal(layer.q_proj.weight, stored[f"layers.{i}.q_proj.weight"])
    assert torch.equal(model.embed_tokens.weight, stored["embed_tokens.weight"])
    # the per-row fallback is read from the scales, not from the config's 48
    expected_group = 64 if case == "int4_packed_g64" else -1
    assert model.layers[0].mlp.w1.group_size == expected_group


def test_another_architecture_is_refused():
    with pytest.raises(RuntimeError, match="state dict mismatch"):
        load_quantized_weights(ToyMoE(layers=1), ref_dir("int4_packed_g64"))


def test_saving_a_loaded_reference_checkpoint_reproduces_it(tmp_path):
    """reference artifact -> this package's load -> this package's save: the same tensors and manifest."""
    model = ToyMoE(seed=5)
    manifest = load_quantized_weights(model, ref_dir("int4_packed_g64"))
    path = save_quantized_checkpoint(model, manifest, str(tmp_path))
    assert os.path.basename(path) == "model-int4.safetensors"
    ours, theirs = load_file(path), load_file(find_weights_file(ref_dir("int4_packed_g64")))
    assert set(ours) == set(theirs)
    assert all(torch.equal(ours[k], theirs[k]) for k in theirs)
    state, again = load_quantized_checkpoint(str(tmp_path))
    assert again.config == manifest.config and again.targets == manifest.targets
    src = json.load(open(tmp_path / SOURCE_FILENAME))
    assert src == {"source_checkpoint": "hf://test/model"}
    assert checkpoint_size_bytes(str(tmp_path)) == sum(os.path.getsize(tmp_path / f) for f in os.listdir(tmp_path))
