"""GPU parity of QuantLinear / lq_quant_linear (the packed W8A16 / W4A16 dense GEMM).

The reference module computes ``F.linear(x.bf16, dequantize_weight())``
(runtime/linear.py:127-131).  Its own kernel tests (tests/unit/test_w8a16_kernel.py:33-82)
hold a packed GEMM to the fp32 truth ``x . dequant(W)^T``: relative L2 error
below 3e-3 (the bf16 output-rounding floor) and no more than 1.2x that of the
BLAS product on the same dequantized weight.  The same bars apply here, to
each GEMM family, with the dequantized weight taken from the CPU oracle
(bit-exact restatement of dequantize_tensor).  With few rows the general
family splits K into slices whose partial sums the combine adds in order,
so the families differ in summation order; each call is deterministic.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from llada_quant_amd.algorithms.symmetric import quantize_tensor
from llada_quant_amd.runtime.linear import QuantLinear, quant_linear
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def oracle_weight(q) -> torch.Tensor:
    """The reference's dequantized bf16 weight, from the CPU oracle, as fp64."""
    d = O.dequant(q.q.cpu().numpy(), q.scale.cpu().numpy(), q.bits, q.group_size, q.logical_shape[-1])
    return torch.from_numpy((d.astype(np.uint32) << 16).view(np.float32)).double()


def rel(out: torch.Tensor, truth: torch.Tensor) -> float:
    return ((out.double().cpu() - truth).norm() / truth.norm()).item()


@pytest.mark.parametrize("M,K,N,bits,group", [
    (1, 512, 256, 8, 128),     # one row: the general kernel
    (7, 1024, 384, 4, 64),     # ragged M, group 64 (per-lane scales)
    (33, 512, 512, 4, 128),    # the wide kernel with a partial row tile
    (129, 2048, 2048, 8, 128),  # test_w8a16_kernel.py's shape at a ragged M
    (300, 1024, 768, 4, 128),
    (16, 512, 256, 8, -1),     # one group per row
    (2, 8192, 512, 4, 128),    # long K: 16 K slices per item
    (160, 1536, 256, 8, 512),  # wide, 2 K slices: the slice boundary at K=768 falls inside group 1
    (200, 1024, 512, 4, 64),   # wide with per-lane scales (two groups per 128-wide chunk)
])
def test_quant_linear_matches_truth_and_blas(dev, M, K, N, bits, group):
    g = torch.Generator().manual_seed(M + K + N)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    q = quantize_tensor(w, bits=bits, group_size=group)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    wd = oracle_weight(q)
    assert torch.equal(wd.float().to(torch.bfloat16).to(dev), q.dequantize(torch.bfloat16))
    truth = x.double().cpu() @ wd.t()
    out = quant_linear(x, q.q, q.scale, bits, group)
    assert out.shape == (M, N) and out.dtype == torch.bfloat16
    blas = x @ q.dequantize(torch.bfloat16).t().contiguous()  # bf16 BLAS product, contiguous operands
    err_blas = rel(blas, truth)
    runs = {"auto": out, "general": quant_linear(x, q.q, q.scale, bits, group, general_kernel=True)}
    if K % 256 == 0 and N % 256 == 0:
        runs["wide"] = quant_linear(x, q.q, q.scale, bits, group, wide_kernel=True)
    for name, o in runs.items():
        err = rel(o, truth)
        assert err < 3e-3, f"{name}: relative L2 error {err:.2e}"
        assert err <= 1.2 * err_blas + 1e-6, f"{name}: {err:.2e} against the BLAS product's {err_blas:.2e}"
    assert torch.equal(out, quant_linear(x, q.q, q.scale, bits, group))  # deterministic


@pytest.mark.parametrize("M,K,N,bits,group", [
    (1, 8192, 512, 8, 128),    # 16 K slices of 4 chunks (16 waves, 2 chunks in flight)
    (16, 8192, 8192, 4, 128),  # the benchmark's shape: 8 slices of 8 chunks (4 in flight)
    (5, 2048, 256, 8, 64),     # per-lane scales, 16 slices of one chunk
    (17, 1024, 384, 4, 32),    # two row tiles, the second with one row
    (20, 2048, 8192, 8, 128),  # two row tiles, 8 slices of 2 chunks
    (32, 1024, 256, 8, -1),    # two full row tiles, one group per row
    (9, 1152, 128, 4, 128),    # 9 chunks: odd, one K slice
    (32, 4096, 256, 8, 128),   # 16 slices with two row tiles: the general path itself
])
def test_small_linear_matches_the_general_path_bit_for_bit(dev, M, K, N, bits, group):
    """Up to 16 rows (32 with at most 8 K slices) take the one-launch kernel, which sums the
    general path's K slices in its order."""
    g = torch.Generator().manual_seed(7 * M + K + N)
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    q = quantize_tensor(w, bits=bits, group_size=group)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(dev)
    out = quant_linear(x, q.q, q.scale, bits, group)
    ref = quant_linear(x, q.q, q.scale, bits, group, general_kernel=True)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    truth = x.double().cpu() @ oracle_weight(q).t()
    assert rel(out, truth) < 3e-3


def test_quant_linear_module_from_linear(dev):
    """QuantLinear.from_linear + forward with bias, leading batch dims, storage bytes."""
    torch.manual_seed(3)
    lin = torch.nn.Linear(1024, 512, bias=True).to(dev)
    with torch.no_grad():
        lin.weight.mul_(0.5)
    ql = QuantLinear.from_linear(lin, bits=4, group_size=128, scale_search="mse", search_grid=16)
    assert ql.qweight.shape == (512, 512) and ql.scale.shape == (512, 8)
    assert ql.storage_bytes() == 512 * 512 + 512 * 8 * 4 + 512 * 2
    assert "packed=True" in ql.extra_repr()
    x = torch.randn(2, 40, 1024, device=dev)
    out = ql(x)
    assert out.shape == (2, 40, 512) and out.dtype == torch.bfloat16
    ref = torch.nn.functional.linear(x.to(torch.bfloat16).float(), ql.dequantize_weight().float()).to(torch.bfloat16)
    ref = ref + ql.bias
    d = (out.float() - ref.float()).abs()
    assert d.max().item() < 2e-2 and (d.sum() / ref.float().abs().sum()).item() < 5e-3


def test_quant_linear_errors(dev):
    q = quantize_tensor((torch.randn(256, 512) * 0.02).to(torch.bfloat16).to(dev), bits=8, group_size=128)
    x = torch.randn(4, 512, device=dev).to(torch.bfloat16)
    with pytest.raises(ValueError, match="input features"):
        quant_linear(x[:, :256], q.q, q.scale, 8, 128)
    with pytest.raises(ValueError, match="bits must be"):
        QuantLinear(512, 256, bits=3)
    with pytest.raises(ValueError, match="even"):
        QuantLinear(511, 256, bits=4)
    with pytest.raises(ValueError, match="exclude each other"):
        quant_linear(x, q.q, q.scale, 8, 128, wide_kernel=True, general_kernel=True)
    q2 = quantize_tensor((torch.randn(128, 512) * 0.02).to(torch.bfloat16).to(dev), bits=8, group_size=128)
    with pytest.raises(NotImplementedError, match="wide kernels need"):  # 128 output features: no whole wide item
        quant_linear(x, q2.q, q2.scale, 8, 128, wide_kernel=True)
    assert quant_linear(x[:0], q.q, q.scale, 8, 128).shape == (0, 256)
