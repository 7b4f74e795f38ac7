"""GPU: the allocation-free layer entry point (lq_moe_layer_noalloc) gives the
same output and routing as lq_moe_layer with a caller-allocated workspace.

Two calls in a row through the C-ABI, the second with fewer tokens, so the
second runs on the static array the first left behind.  Both entry points
launch the same kernels on the same inputs, so the comparison is bit-exact.
"""

from __future__ import annotations

import pytest
import torch

from llada_quant_amd.runtime import _lib
from llada_quant_amd.runtime.fused_moe import workspace_bytes
from test_gpu_moe import make_layer

pytestmark = pytest.mark.gpu


def _args(x, logits, q1, q2, k, flags):
    T, H = x.shape
    E, two_i, _ = q1.logical_shape
    return (_lib.ptr(x), _lib.ptr(logits), _lib.LQ_F32, T, H, two_i // 2, E, k, 1,
            _lib.ptr(q1.q), _lib.ptr(q1.scale), _lib.ptr(q2.q), _lib.ptr(q2.scale), q1.bits,
            q1.group_size, q2.group_size, flags)


def _with_workspace(x, logits, q1, q2, k, flags):
    T, H = x.shape
    E, two_i, _ = q1.logical_shape
    ws = _lib.moe_workspace(workspace_bytes(T, H, two_i // 2, E, k), x.device)
    out = torch.empty_like(x)
    ids = torch.empty(T, k, dtype=torch.int32, device=x.device)
    rc = _lib.load().lq_moe_layer(*_args(x, logits, q1, q2, k, flags), _lib.ptr(ws), ws.numel(), _lib.ptr(out),
                                  _lib.ptr(ids), _lib.stream(x.device))
    _lib.check(rc, "moe_layer")
    return out, ids


def _no_alloc(x, logits, q1, q2, k, flags):
    T, _ = x.shape
    out = torch.empty_like(x)
    ids = torch.empty(T, k, dtype=torch.int32, device=x.device)
    rc = _lib.load().lq_moe_layer_noalloc(*_args(x, logits, q1, q2, k, flags), _lib.ptr(out), _lib.ptr(ids),
                                          _lib.stream(x.device))
    _lib.check(rc, "moe_layer_noalloc")
    return out, ids


@pytest.mark.parametrize("flags", [0, _lib.LQ_MOE_FUSED_LAYER], ids=["default", "fused_layer"])
@pytest.mark.parametrize("bits", [4, 8])
def test_no_alloc_layer_matches_workspace_layer(dev, bits, flags):
    """E=64, H=2048, I=1024, top-8: 64 tokens, then 24 on the same static array."""
    q1, q2 = make_layer(dev, 64, 2048, 1024, bits, seed=70 + bits, search="mse", grid=16)
    g = torch.Generator().manual_seed(71)
    for T in (64, 24):
        x = torch.randn(T, 2048, generator=g).to(torch.bfloat16).to(dev)
        logits = torch.randn(T, 64, generator=g).to(dev)
        ref_out, ref_ids = _with_workspace(x, logits, q1, q2, 8, flags)
        out, ids = _no_alloc(x, logits, q1, q2, 8, flags)
        torch.cuda.synchronize()
        assert torch.equal(ids, ref_ids), f"T={T}: routing differs"
        assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16)), f"T={T}: output differs"


def test_no_alloc_layer_rejects_a_layer_beyond_the_static_array(dev):
    """4096 tokens x top-8 x H=2048 need more than the 64 MiB array: a clear error, nothing launched."""
    q1, q2 = make_layer(dev, 8, 2048, 1024, 4, seed=72)
    x = torch.zeros(4096, 2048, dtype=torch.bfloat16, device=dev)
    logits = torch.zeros(4096, 8, device=dev)
    with pytest.raises(NotImplementedError, match="scratch"):
        _no_alloc(x, logits, q1, q2, 8, 0)
