"""The C-ABI library without a GPU: it loads, exports every declared symbol, and
rejects bad arguments on the host before any device work.

These tests make no compute call.  The host-side validation they exercise is
the same code every GPU call runs first; its messages are the substrings the
reference's tests match on (tests/unit/test_int4.py, test_scale_search.py).
"""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from llada_quant_amd.runtime import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "lladaq.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lq_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_entry_points():
    names = declared_functions()
    assert names, "no lq_* declarations found"
    assert set(names) == set(_lib.SIGNATURES), (
        f"header and ctypes binding disagree: only in header {set(names) - set(_lib.SIGNATURES)}, "
        f"only in binding {set(_lib.SIGNATURES) - set(names)}")


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True, check=True)
    exported = {line.split()[-1] for line in out.stdout.splitlines() if line.strip()}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing


def test_abi_version():
    assert _lib.load().lq_abi_version() == _lib.ABI_VERSION


NULL = ctypes.c_void_p(0)


def _rc_and_msg(rc):
    return rc, _lib.load().lq_last_error().decode()


def test_bad_bits_are_rejected_on_the_host():
    lib = _lib.load()
    rc, msg = _rc_and_msg(lib.lq_dequant(NULL, NULL, _lib.LQ_F32, 4, 8, 3, 128, NULL, _lib.LQ_BF16, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "bits must be 8 or 4" in msg
    rc, msg = _rc_and_msg(lib.lq_quantize(NULL, _lib.LQ_F32, 4, 8, 5, 1, 128, 0, 24, 0.5, NULL, NULL,
                                          _lib.LQ_F32, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "bits must be 8 or 4" in msg


def test_int4_layout_errors_use_the_reference_messages():
    lib = _lib.load()
    rc, msg = _rc_and_msg(lib.lq_pack_int4(NULL, 2, 3, NULL, NULL, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "even" in msg
    rc, msg = _rc_and_msg(lib.lq_quantize(NULL, _lib.LQ_F32, 2, 7, 4, 1, -1, 0, 24, 0.5, NULL, NULL,
                                          _lib.LQ_F32, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "even last dimension" in msg
    rc, msg = _rc_and_msg(lib.lq_quantize(NULL, _lib.LQ_F32, 2, 96, 4, 1, 3, 0, 24, 0.5, NULL, NULL,
                                          _lib.LQ_F32, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "even group_size" in msg


def test_scale_search_argument_errors():
    lib = _lib.load()
    rc, msg = _rc_and_msg(lib.lq_search_group_scale(NULL, _lib.LQ_F32, 4, 128, 4, 0, 0.5, NULL, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "grid must be >= 1" in msg
    rc, msg = _rc_and_msg(lib.lq_search_group_scale(NULL, _lib.LQ_F32, 4, 128, 4, 8, 1.0, NULL, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "max_shrink must lie in" in msg
    rc, msg = _rc_and_msg(lib.lq_quantize(NULL, _lib.LQ_F32, 4, 128, 8, 1, 128, 7, 24, 0.5, NULL, NULL,
                                          _lib.LQ_F32, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "scale_search must be" in msg


def test_router_and_permute_argument_errors():
    lib = _lib.load()
    rc, msg = _rc_and_msg(lib.lq_route_topk(NULL, _lib.LQ_F32, 4, 64, 65, 0, NULL, NULL, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "k" in msg
    rc, msg = _rc_and_msg(lib.lq_route_topk(NULL, _lib.LQ_F32, 4, 300, 8, 0, NULL, NULL, NULL))
    assert rc == _lib.LQ_ERR_UNSUPPORTED
    rc, msg = _rc_and_msg(lib.lq_moe_permute(NULL, 4, 2, 0, NULL, NULL, NULL, NULL))
    assert rc == _lib.LQ_ERR_UNSUPPORTED


def test_empty_inputs_are_no_ops_without_device_work():
    lib = _lib.load()
    assert lib.lq_route_topk(NULL, _lib.LQ_F32, 0, 64, 8, 0, NULL, NULL, NULL) == _lib.LQ_OK
    assert lib.lq_unpack_int4(NULL, 0, 16, NULL, NULL) == _lib.LQ_OK
    assert lib.lq_dequant(NULL, NULL, _lib.LQ_F32, 0, 128, 4, 128, NULL, _lib.LQ_BF16, NULL) == _lib.LQ_OK


def test_moe_workspace_size_is_monotone_in_tokens_and_covers_the_buffers():
    lib = _lib.load()
    sizes = [lib.lq_moe_workspace_bytes(T, 2048, 1024, 64, 8) for T in (1, 64, 512, 4096)]
    assert sizes == sorted(sizes) and sizes[0] > 0
    # at least the bf16 gate / up rows [T*k, 2I] and the bf16 slot outputs [T*k, H]
    T, H, I, k = 512, 2048, 1024, 8
    assert sizes[2] >= T * k * (2 * I * 2 + H * 2)
    assert lib.lq_moe_workspace_bytes(-1, 2048, 1024, 64, 8) == 0


def test_moe_forward_rejects_unsupported_shapes_on_the_host():
    lib = _lib.load()
    ws = lib.lq_moe_workspace_bytes(8, 100, 64, 4, 2)
    rc, msg = _rc_and_msg(lib.lq_moe_forward(NULL, 8, 100, 64, 4, 2, NULL, NULL, NULL, NULL, 4, 128, 128, 0, NULL,
                                             NULL, NULL, ws, NULL, NULL))
    assert rc == _lib.LQ_ERR_UNSUPPORTED and "hidden" in msg
    rc, msg = _rc_and_msg(lib.lq_moe_forward(NULL, 8, 128, 64, 4, 5, NULL, NULL, NULL, NULL, 4, 128, 128, 0, NULL,
                                             NULL, NULL, ws, NULL, NULL))
    assert rc == _lib.LQ_ERR_VALUE and "top_k" in msg


# ---------------------------------------------------------------------------
# Python host logic that runs before any kernel
# ---------------------------------------------------------------------------


def test_quant_config_validation_messages():
    from llada_quant_amd import ExecutionMode, QuantConfig

    assert QuantConfig().mode is ExecutionMode.PACKED
    with pytest.raises(ValueError, match="bits must be 8 or 4"):
        QuantConfig(bits=3)
    with pytest.raises(ValueError, match="even group_size"):
        QuantConfig(bits=4, group_size=33)
    with pytest.raises(ValueError, match="scale_search"):
        QuantConfig(scale_search="best")
    with pytest.raises(ValueError, match="search_grid"):
        QuantConfig(search_grid=0)
    cfg = QuantConfig(bits=4, scale_search="mse", search_grid=16)
    assert QuantConfig.from_dict(cfg.to_dict()) == cfg


def test_compute_on_cpu_tensors_fails_loudly():
    """No CPU fallback: the product path raises for tensors that are not on a HIP device."""
    from llada_quant_amd.algorithms.symmetric import dequantize_tensor, quantize_tensor

    w = torch.randn(4, 256).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        quantize_tensor(w, bits=4, group_size=128)
    with pytest.raises(RuntimeError, match="GPU"):
        dequantize_tensor(torch.zeros(4, 128, dtype=torch.int8), torch.ones(4, 2), 4, 128, torch.bfloat16,
                          packed=True)


def test_int4_layout_validation_runs_on_the_host():
    from llada_quant_amd.algorithms.symmetric import quantize_tensor

    with pytest.raises(ValueError, match="even last dimension"):
        quantize_tensor(torch.randn(4, 7), bits=4, group_size=-1)
    with pytest.raises(ValueError, match="even group_size"):
        quantize_tensor(torch.randn(4, 96), bits=4, group_size=3)


def test_token_chunks_cover_calls_within_the_32bit_bounds():
    """Layers above one call's addressing bound (T*k*max(2I, H)*2 < 2^31) are split into
    even token chunks: C5's 32768 tokens at top-8, H 2048, I 1024 are one call; 131072 tokens
    would be three."""
    from llada_quant_amd.runtime.fused_moe import _chunks, max_tokens_per_call

    lim = max_tokens_per_call(2048, 1024, 8)
    assert lim == (2**31 - 1) // (8 * 2048 * 2) == 65535
    assert _chunks(32768, lim) == [(0, 32768)]
    assert _chunks(131072, lim) == [(0, 43690), (43690, 87381), (87381, 131072)]
    assert max_tokens_per_call(1024, 4096, 8) == (2**31 - 1) // (8 * 8192 * 2)  # 2I above H
    for T, lim in [(1, 5), (10, 3), (17, 17), (18, 17), (1000, 7)]:
        spans = _chunks(T, lim)
        assert spans[0][0] == 0 and spans[-1][1] == T
        assert all(a1 == b0 for (_, a1), (b0, _) in zip(spans, spans[1:]))
        assert all(0 < c1 - c0 <= lim for c0, c1 in spans)
        assert max(c1 - c0 for c0, c1 in spans) - min(c1 - c0 for c0, c1 in spans) <= 1
    assert max_tokens_per_call(64, 64, 1) == 1 << 18


def test_no_alloc_layer_rejects_a_layer_beyond_its_static_array_on_the_host():
    """lq_moe_layer_noalloc's scratch limit is checked before any device call."""
    lib = _lib.load()
    rc, msg = _rc_and_msg(lib.lq_moe_layer_noalloc(NULL, NULL, _lib.LQ_F32, 4096, 2048, 1024, 8, 8, 0, NULL, NULL,
                                                   NULL, NULL, 4, 128, 128, 0, NULL, NULL, NULL))
    assert rc == _lib.LQ_ERR_UNSUPPORTED and "scratch" in msg and "lq_moe_layer" in msg
