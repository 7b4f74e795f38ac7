"""Packed checkpoints straight to the GPU (formats/safetensors.py:102-167 of the reference).

A PACKED model saved to ``model-int{bits}.safetensors`` + ``quantization.json`` stores
only codes and scales (never the BF16 w1/w2, formats/safetensors.py:42-65); a plain
model loading it on the GPU gets the packed buffers in device memory, bit-identical to
the saved ones, its expert blocks re-wired to them, and the same fused_moe output.
"""

from __future__ import annotations

import os

import pytest
import torch
from safetensors import safe_open

from conftest import TinyMoEModel
from llada_quant_amd import ExecutionMode, QuantConfig, fused_moe, quantize_model
from llada_quant_amd.checkpoint import load_quantized_weights, save_quantized_checkpoint
from llada_quant_amd.runtime.moe import PackedExpertTensor, is_packed_expert_block
from llada_quant_amd.runtime.routing import route_topk

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [4, 8])
def test_packed_checkpoint_round_trip_to_gpu(dev, tmp_path, bits):
    torch.manual_seed(0)
    model = TinyMoEModel().to(dev)
    result = quantize_model(model, QuantConfig(bits=bits, group_size=64, execution_mode=ExecutionMode.PACKED.value))
    path = save_quantized_checkpoint(model, result, str(tmp_path))
    assert os.path.basename(path) == f"model-int{bits}.safetensors"
    assert os.path.exists(tmp_path / "quantization.json")
    with safe_open(path, framework="pt") as f:
        keys = set(f.keys())
    assert "layers.0.mlp._qw1" in keys and "layers.1.mlp._sw2" in keys
    assert not any(k.endswith("mlp.w1") or k.endswith("mlp.w2") for k in keys)

    fresh = TinyMoEModel(seed=123)  # plain, on the CPU, different BF16 weights
    manifest = load_quantized_weights(fresh, str(tmp_path), device=dev)
    assert manifest["config"]["bits"] == bits
    for i in range(2):
        a, b = model.layers[i].mlp, fresh.layers[i].mlp
        assert is_packed_expert_block(b)
        for name in ("_qw1", "_sw1", "_qw2", "_sw2"):
            assert getattr(b, name).device.type == "cuda"
            assert torch.equal(getattr(a, name), getattr(b, name))
        assert isinstance(b.w1, PackedExpertTensor)
        assert torch.equal(a.w1, b.w1) and torch.equal(a.w2, b.w2)  # dequantized through the HIP kernel
    g = torch.Generator().manual_seed(1)
    x = torch.randn(24, model.layers[0].mlp._qw1.shape[-1] * (2 if bits == 4 else 1), generator=g)
    x = x.to(torch.bfloat16).to(dev)
    probs = torch.softmax(torch.randn(24, model.layers[0].mlp._qw1.shape[0], generator=g), -1).to(dev)
    ids, _ = route_topk(probs.log(), 2)
    for i in range(2):
        ya = fused_moe(x, model.layers[i].mlp.w1, model.layers[i].mlp.w2, probs, ids)
        yb = fused_moe(x, fresh.layers[i].mlp.w1, fresh.layers[i].mlp.w2, probs, ids)
        assert torch.equal(ya, yb)
    assert torch.equal(model.layers[0].q_proj.weight, fresh.layers[0].q_proj.weight)


def test_checkpoint_of_another_architecture_is_rejected(dev, tmp_path):
    torch.manual_seed(0)
    model = TinyMoEModel().to(dev)
    result = quantize_model(model, QuantConfig(bits=8, group_size=64, execution_mode=ExecutionMode.PACKED.value))
    save_quantized_checkpoint(model, result, str(tmp_path))
    with pytest.raises(RuntimeError, match="mismatch"):
        load_quantized_weights(TinyMoEModel(layers=1), str(tmp_path), device=dev)
