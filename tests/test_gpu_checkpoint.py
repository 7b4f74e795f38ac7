"""Packed checkpoints on the GPU: reference-written artifacts and this package's own.

The reference artifacts (``tests/golden/ckpt_*``, written by LLaDA_Quant
v0.2.0's ``quantize_model`` + ``save_quantized_checkpoint``) load straight into
device memory, and the expert weights this package derives from them --
``block.w1`` / ``block.w2`` through the HIP dequant kernel, PACKED or
REFERENCE -- are bit for bit what the reference's blocks returned (SHA-256 of
the BF16 bytes, tests/golden/make_ckpt_golden.py).  This package's own
artifacts round-trip in both modes, with the per-row group fallback (the
cases of tests/unit/test_checkpoint_format.py:115-175), and hold no BF16 expert
weights (:42-65).
"""

from __future__ import annotations

import hashlib
import os

import numpy as np
import pytest
import torch
from safetensors import safe_open

from conftest import ToyMoE, bits_u16
from llada_quant_amd import (
    ExecutionMode,
    QuantConfig,
    QuantizationManifest,
    fused_moe,
    load_quantized_weights,
    quantize_model,
    save_quantized_checkpoint,
)
from llada_quant_amd.runtime.moe import PackedExpertTensor, is_packed_expert_block
from llada_quant_amd.runtime.routing import route_topk

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _save(model, config, directory):
    result = quantize_model(model, config)
    manifest = QuantizationManifest(source_checkpoint="hf://test/model", config=config, targets=result.targets)
    return result, save_quantized_checkpoint(model, manifest, directory)


@pytest.mark.parametrize("case", ["int4_packed_g64", "int8_reference_g64", "int8_packed_g48"])
def test_reference_checkpoint_dequantizes_to_the_reference_bits(dev, case):
    directory = os.path.join(GOLDEN, f"ckpt_{case}")
    expect = np.load(os.path.join(directory, "expected.npz"))
    model = ToyMoE(seed=77)
    manifest = load_quantized_weights(model, directory, device=dev)
    packed = manifest.config.mode is ExecutionMode.PACKED
    for i, layer in enumerate(model.layers):
        block = layer.mlp
        assert is_packed_expert_block(block) == packed
        assert block._qw1.device.type == "cuda"
        for w in ("w1", "w2"):
            t = getattr(block, w)
            assert isinstance(t, PackedExpertTensor) == packed
            got = bits_u16(t if not packed else t.materialize())
            assert tuple(got.shape) == tuple(expect[f"layer{i}_{w}_shape"])
            assert np.array_equal(got.reshape(-1)[:64], expect[f"layer{i}_{w}_head"])
            assert hashlib.sha256(got.tobytes()).digest() == expect[f"layer{i}_{w}_sha256"].tobytes()


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("mode", [ExecutionMode.PACKED, ExecutionMode.REFERENCE])
def test_own_checkpoint_round_trip(dev, tmp_path, bits, mode):
    torch.manual_seed(0)
    model = ToyMoE().to(dev)
    config = QuantConfig(bits=bits, group_size=64, targets=("expert",), execution_mode=mode.value)
    _, path = _save(model, config, str(tmp_path))
    assert os.path.basename(path) == f"model-int{bits}.safetensors"
    with safe_open(path, framework="pt") as f:
        keys = set(f.keys())
    assert "layers.0.mlp._qw1" in keys and "layers.1.mlp._sw2" in keys
    assert not [k for k in keys if k.endswith(("mlp.w1", "mlp.w2"))], "BF16 expert weights were stored"

    fresh = ToyMoE(seed=123)  # plain, on the host, different BF16 weights
    manifest = load_quantized_weights(fresh, str(tmp_path), device=dev)
    assert manifest.config == config
    for a, b in ((m.mlp, f.mlp) for m, f in zip(model.layers, fresh.layers)):
        assert is_packed_expert_block(b) == (mode is ExecutionMode.PACKED)
        for name in ("_qw1", "_sw1", "_qw2", "_sw2"):
            assert getattr(b, name).device.type == "cuda"
            assert torch.equal(getattr(a, name), getattr(b, name))
        assert torch.equal(a.w1, b.w1) and torch.equal(a.w2, b.w2)
    assert torch.equal(model.layers[0].q_proj.weight, fresh.layers[0].q_proj.weight)
    if mode is ExecutionMode.PACKED:
        g = torch.Generator().manual_seed(1)
        x = torch.randn(24, 128, generator=g).to(torch.bfloat16).to(dev)
        probs = torch.softmax(torch.randn(24, 4, generator=g), -1).to(dev)
        ids, _ = route_topk(probs.log(), 2)
        for i in range(2):
            ya = fused_moe(x, model.layers[i].mlp.w1, model.layers[i].mlp.w2, probs, ids)
            yb = fused_moe(x, fresh.layers[i].mlp.w1, fresh.layers[i].mlp.w2, probs, ids)
            assert torch.equal(ya, yb)


def test_group_fallback_is_recovered_from_the_scales(dev, tmp_path):
    """48 does not divide K=128: one scale per row at save time; the reload follows the scales."""
    torch.manual_seed(0)
    model = ToyMoE().to(dev)
    _save(model, QuantConfig(bits=8, group_size=48, targets=("expert",)), str(tmp_path))
    assert model.layers[0].mlp._sw1.shape[-1] == 1
    fresh = ToyMoE(seed=5)
    load_quantized_weights(fresh, str(tmp_path), device=dev)
    assert fresh.layers[0].mlp.w1.group_size == -1
    assert torch.equal(fresh.layers[0].mlp.w1, model.layers[0].mlp.w1)


def test_forward_after_reload_matches_forward_before_save(dev, tmp_path):
    torch.manual_seed(0)
    model = ToyMoE().to(dev)
    _save(model, QuantConfig(bits=8, group_size=64, targets=("expert",)), str(tmp_path))
    x = torch.randn(5, 128, dtype=torch.bfloat16)
    before = model.layers[0].mlp(x)
    fresh = ToyMoE(seed=3)
    load_quantized_weights(fresh, str(tmp_path), device=dev)
    assert torch.equal(fresh.layers[0].mlp(x), before)


def test_strict_load_catches_a_real_mismatch(dev, tmp_path):
    torch.manual_seed(0)
    model = ToyMoE().to(dev)
    _save(model, QuantConfig(bits=8, group_size=64, targets=("expert",)), str(tmp_path))
    with pytest.raises(RuntimeError, match="state dict mismatch"):
        load_quantized_weights(ToyMoE(layers=1), str(tmp_path), device=dev)
    # a model with an extra tensor the checkpoint lacks: missing key, strict raises, non-strict loads
    extra = ToyMoE(seed=9)
    extra.layers[0].register_buffer("calibration", torch.zeros(3), persistent=True)
    with pytest.raises(RuntimeError, match="missing=\\['layers.0.calibration'\\]"):
        load_quantized_weights(extra, str(tmp_path), device=dev)
    load_quantized_weights(extra, str(tmp_path), strict=False, device=dev)
    assert torch.equal(extra.layers[1].mlp._qw2, model.layers[1].mlp._qw2)
