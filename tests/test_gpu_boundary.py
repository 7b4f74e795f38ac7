"""The PACKED residency boundary: ``block.w1`` / ``block.w2`` and quantize_model.

Ports of the reference's boundary-semantics tests
(tests/unit/test_llada_moe_adapter.py:30-138, test_memory.py:33-156,
test_int4.py:229-254 of LLaDA_Quant v0.2.0) onto the GPU path: quantization
runs through the HIP quantizer and every ``block.w1`` materialization through
the HIP dequant kernel.
"""

from __future__ import annotations

import copy

import pytest
import torch

from conftest import ExpertMLP, ToyMoE
from llada_quant_amd import ExecutionMode, PackedExpertTensor, QuantConfig, fused_moe, quantize_model
from llada_quant_amd.adapters.llada_moe import (
    describe_fused_expert_block,
    quantize_llada_experts,
    restore_llada_experts_from_buffers,
)
from llada_quant_amd.algorithms.symmetric import dequantize_tensor
from llada_quant_amd.runtime import moe as moe_module
from llada_quant_amd.runtime.moe import (
    is_packed_expert_block,
    materialize_expert_params,
    quant_result_from_buffers,
    quantize_fused_experts,
)
from llada_quant_amd.runtime.routing import route_topk

pytestmark = pytest.mark.gpu


def _config(bits=8, group_size=64, mode=ExecutionMode.PACKED, **kw):
    return QuantConfig(bits=bits, group_size=group_size, targets=("expert",), execution_mode=mode.value, **kw)


def test_quantization_leaves_the_router_bit_identical(expert_block):
    original = expert_block.gate.weight.detach().clone()
    quantize_llada_experts(expert_block, _config())
    assert torch.equal(expert_block.gate.weight, original)


def test_packed_mode_shapes_and_error_budget(expert_block):
    original = expert_block.w1.detach().clone()
    records = quantize_llada_experts(expert_block, _config())
    assert len(records) == 1 and records[0].name == ""
    assert is_packed_expert_block(expert_block)
    assert isinstance(expert_block.w1, PackedExpertTensor)
    assert expert_block.w1.shape == original.shape
    assert expert_block.w1.dtype == torch.bfloat16
    assert expert_block._sw1.shape == (4, 128, 2)
    error = (expert_block.w1.float() - original.float()).abs()
    assert error.max() < original.abs().max() / 127 * 1.1


def test_reference_mode_keeps_parameters_and_matches_packed_values(expert_block):
    packed = copy.deepcopy(expert_block)
    reference = copy.deepcopy(expert_block)
    quantize_llada_experts(packed, _config(mode=ExecutionMode.PACKED))
    quantize_llada_experts(reference, _config(mode=ExecutionMode.REFERENCE))
    assert is_packed_expert_block(packed) and not is_packed_expert_block(reference)
    assert torch.equal(packed.w1, reference.w1), "both modes must dequantize identically"
    assert torch.equal(packed._qw1, reference._qw1)


def test_quantization_is_reproducible(dev):
    a, b = ExpertMLP().to(dev), ExpertMLP().to(dev)
    quantize_llada_experts(a, _config())
    quantize_llada_experts(b, _config())
    for attr in ("_qw1", "_sw1", "_qw2", "_sw2"):
        assert torch.equal(getattr(a, attr), getattr(b, attr))
    assert torch.equal(a.w1, b.w1)


def test_dequantization_happens_per_access_not_once(expert_block):
    """Each access is a fresh handle; each materialization fresh memory (no cached BF16 copy)."""
    quantize_llada_experts(expert_block, _config())
    first, second = expert_block.w1, expert_block.w1
    assert first is not second
    assert torch.equal(first, second)
    a, b = first.materialize(), first.materialize()
    assert a.data_ptr() != b.data_ptr()


def test_materialize_refuses_to_write_into_a_packed_block(expert_block):
    weights = quantize_fused_experts(expert_block.w1.detach(), expert_block.w2.detach(), bits=8, group_size=64)
    quantize_llada_experts(expert_block, _config())
    with pytest.raises(RuntimeError, match="cannot be assigned"):
        materialize_expert_params(expert_block, weights)


def test_restore_reinstalls_access_after_a_bare_buffer_load(expert_block):
    quantize_llada_experts(expert_block, _config())
    expected = expert_block.w1.clone()
    delattr(expert_block, "_llada_quant_meta")
    with pytest.raises(RuntimeError, match="Reload through"):
        _ = expert_block.w1
    assert restore_llada_experts_from_buffers(expert_block, _config()) == 1
    assert torch.equal(expert_block.w1, expected)


def test_quant_result_from_buffers_derives_the_group_size(dev):
    w1 = torch.randn(2, 8, 128, device=dev) * 0.02
    w2 = torch.randn(2, 128, 4, device=dev) * 0.02
    weights = quantize_fused_experts(w1, w2, bits=8, group_size=64)
    rebuilt = quant_result_from_buffers(weights.w1.q, weights.w1.scale, 8)
    assert rebuilt.group_size == 64 and rebuilt.logical_shape == (2, 8, 128)
    assert torch.equal(rebuilt.dequantize(torch.float32), weights.w1.dequantize(torch.float32))
    fallback = quantize_fused_experts(torch.randn(2, 4, 100, device=dev), torch.randn(2, 4, 100, device=dev),
                                      bits=8, group_size=64).w1
    assert fallback.group_size == -1
    assert quant_result_from_buffers(fallback.q, fallback.scale, 8).group_size == -1


def test_expert_block_shape_reports_element_count(dev):
    shape = describe_fused_expert_block(ExpertMLP().to(dev))
    assert shape.numel == 4 * (2 * 64 * 128 + 128 * 64)
    assert "E=4" in shape.describe()


def test_packed_mode_removes_the_bf16_parameters(moe_model):
    quantize_model(moe_model, _config())
    for layer in moe_model.layers:
        names = dict(layer.mlp.named_parameters())
        assert "w1" not in names and "w2" not in names
        assert is_packed_expert_block(layer.mlp)
        assert layer.mlp.w1.shape == (4, 128, 128) and layer.mlp.w1.dtype == torch.bfloat16
    keys = set(moe_model.state_dict())
    assert not [k for k in keys if k.endswith(("mlp.w1", "mlp.w2"))]
    assert {"layers.0.mlp._qw1", "layers.0.mlp._sw1"} <= keys


def test_packed_weights_are_read_only(moe_model):
    quantize_model(moe_model, _config())
    with pytest.raises(AttributeError):
        moe_model.layers[0].mlp.w1 = torch.zeros(1)


def test_in_place_weight_loaders_are_blocked_in_packed_mode(moe_model):
    loaded = []
    ExpertMLP.load_state_dict_from_unfused = lambda self, src: loaded.append(src)
    moe_module._PACKED_CLASSES.clear()
    try:
        moe_model.layers[0].mlp.load_state_dict_from_unfused("before")
        assert loaded == ["before"]
        quantize_model(moe_model, _config())
        with pytest.raises(RuntimeError, match="silently discarded"):
            moe_model.layers[0].mlp.load_state_dict_from_unfused("after")
        assert loaded == ["before"]
    finally:
        del ExpertMLP.load_state_dict_from_unfused
        moe_module._PACKED_CLASSES.clear()


def test_int4_adapter_stores_packed_codes(moe_model):
    result = quantize_model(moe_model, _config(bits=4))
    assert all(t.packed for t in result.targets)
    block = moe_model.layers[0].mlp
    assert block._qw1.shape == (4, 128, 64)
    assert block.w1.shape == (4, 128, 128)


def test_int4_and_int8_both_reconstruct_after_a_forward(moe_model):
    x = torch.randn(6, 128, device=moe_model.router.weight.device).to(torch.bfloat16)
    reference = moe_model.layers[0].mlp(x)
    for bits, tolerance in ((8, 0.05), (4, 0.6)):
        clone = copy.deepcopy(moe_model)
        quantize_model(clone, _config(bits=bits))
        out = clone.layers[0].mlp(x)
        relative = (out - reference).abs().max() / reference.abs().max()
        assert relative < tolerance, f"INT{bits} relative error {relative:.3f}"


def test_mse_search_reaches_the_adapter_and_beats_amax(moe_model):
    original = moe_model.layers[0].mlp.w1.float()
    a = copy.deepcopy(moe_model)
    m = copy.deepcopy(moe_model)
    ra = quantize_model(a, _config(bits=4, scale_search="amax"))
    rm = quantize_model(m, _config(bits=4, scale_search="mse"))
    assert ra.quantized_bytes == rm.quantized_bytes
    assert (m.layers[0].mlp.w1.float() - original).norm() < (a.layers[0].mlp.w1.float() - original).norm()


def test_block_w1_feeds_fused_moe_without_a_bf16_copy(moe_model):
    """TritonFusedMoEBlock.forward's call: fused_moe(x, self.w1, self.w2, gating_output, topk_ids)."""
    quantize_model(moe_model, _config(bits=4))
    block = moe_model.layers[0].mlp
    x = torch.randn(9, 128, device=block._qw1.device).to(torch.bfloat16)
    logits = block.gate(x).float()
    probs = torch.softmax(logits, -1, dtype=torch.float32)
    topk_ids = probs.topk(2, dim=-1).indices
    out = fused_moe(x, block.w1, block.w2, probs, topk_ids)
    # the same layer through explicit dequantization (the reference's path), fp32 math
    w1 = dequantize_tensor(block._qw1, block._sw1, 4, 64, torch.bfloat16, packed=True).float()
    w2 = dequantize_tensor(block._qw2, block._sw2, 4, -1, torch.bfloat16, packed=True).float()
    ref = torch.zeros(9, 128, device=x.device)
    for t in range(9):
        for j in range(2):
            e = int(topk_ids[t, j])
            g = (x[t].float() @ w1[e, :64].T).bfloat16().float()
            u = (x[t].float() @ w1[e, 64:].T).bfloat16().float()
            act = (torch.nn.functional.silu(g).bfloat16().float() * u).bfloat16().float()
            ref[t] += probs[t, e] * (act @ w2[e].T)
    assert (out.float() - ref).abs().max() < 2e-2
    assert ((out.float() - ref).abs().sum() / ref.abs().sum()) < 5e-3


def test_cpu_model_fails_loudly():
    """No CPU fallback: quantizing a CPU-resident model raises."""
    model = ToyMoE()
    with pytest.raises(RuntimeError, match="GPU"):
        quantize_model(model, _config())
