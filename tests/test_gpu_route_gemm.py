"""GPU parity of the fused router GEMM + top-k (lq_route_gemm_topk).

The reference routes with ``router_logits = block.gate(x_flat)`` (a bias-free
bf16 nn.Linear) then ``softmax(dtype=float32).topk(k)`` (trajectory/llada.py:228-234).
Pins:
- the bf16 logits differ from the fp64 product by at most one bf16 ulp of the value
  plus the fp32 accumulation bound H * 2^-24 * sum |x w| (cancellation can leave a
  logit near zero whose ulp is smaller than that), and equal the rounded fp64 product
  for at least 99% of entries;
- ids and weights equal route_topk applied to the kernel's own logits, bit for bit
  (the same routing routine);
- against routing of the fp64-exact logits, ids differ only for tokens whose logits
  differ.
"""

from __future__ import annotations

import pytest
import torch

from llada_quant_amd.runtime.routing import route_gemm_topk, route_topk

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H,E,k,renorm", [(64, 2048, 64, 8, False), (1, 1024, 16, 2, True),
                                            (37, 512, 60, 4, False), (4096, 2048, 64, 8, False)])
def test_route_gemm_topk(dev, T, H, E, k, renorm):
    g = torch.Generator().manual_seed(T + E)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(E, H, generator=g) * 0.02).to(torch.bfloat16)
    ids, wts, logits = route_gemm_topk(x.to(dev), w.to(dev), k, renormalize=renorm, return_logits=True)
    prod = x.double() @ w.double().t()
    exact = prod.to(torch.bfloat16)
    got = logits.cpu()
    mag = x.double().abs() @ w.double().abs().t()
    bound = prod.abs() * 2.0**-8 + H * 2.0**-24 * mag
    assert bool(((got.double() - prod).abs() <= bound).all())
    assert float((got == exact).float().mean()) >= 0.99
    ids2, wts2 = route_topk(logits, k, renormalize=renorm)
    assert torch.equal(ids, ids2) and torch.equal(wts, wts2)
    ids_ref, _ = route_topk(exact.to(dev), k, renormalize=renorm)
    rows_equal = (got == exact).all(dim=1).to(dev)
    assert torch.equal(ids[rows_equal], ids_ref[rows_equal])


def test_route_gemm_topk_errors(dev):
    x = torch.randn(4, 256, device=dev).to(torch.bfloat16)
    with pytest.raises(NotImplementedError, match="num_experts <= 64"):
        route_gemm_topk(x, torch.zeros(65, 256, device=dev), 2)
    with pytest.raises(ValueError, match="gate_weight"):
        route_gemm_topk(x, torch.zeros(8, 128, device=dev), 2)
    with pytest.raises(NotImplementedError, match="multiple of 32"):
        route_gemm_topk(x[:, :80].contiguous(), torch.zeros(8, 80, device=dev), 2)
