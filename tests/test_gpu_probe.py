"""Exact end-to-end probes of the grouped GEMM's fragment layout and in-register dequant.

The layer is built so that every product and sum inside the kernel is exact:

* tokens are one-hot: x[t] = e_t;
* W1 gate rows are all 1.0, so g = 1 for every feature and act = a, one
  constant (a = bf16(bf16(silu(1)) * u) with u in {0, 1});
* W1 up rows are one-hot in K: up[n, h] = 1 iff h % I == n, so token t
  activates exactly feature n(t) = t % I;
* W2 row 0 is all 1.0 (it returns a itself); rows h >= 1 hold random codes
  and scales over many binades: y[t, h] = a * W2[h, n(t)], exact in fp32.

So out[t, h] = bf16(a * deq(W2)[h, n(t)]) exactly, with deq the standalone
(software-rounded) dequant kernel: the matrix cores consume the reference's
bf16(fp32(q) * s) weights.  A wrong K pairing in either GEMM, a wrong
token row, or an in-register dequant that rounds differently from
dequantize_tensor changes the output bits.
"""

from __future__ import annotations

import pytest
import torch

from llada_quant_amd.algorithms.symmetric import QuantResult, dequantize_tensor
from llada_quant_amd.runtime.fused_moe import fused_moe_packed

pytestmark = pytest.mark.gpu


def _codes(values: torch.Tensor, bits: int) -> torch.Tensor:
    """int codes [..., K] -> storage (packed two per byte at 4 bits)."""
    v = values.to(torch.int16)
    if bits == 8:
        return v.to(torch.int8)
    lo, hi = v[..., 0::2] & 0x0F, v[..., 1::2] & 0x0F
    return (lo | (hi << 4)).to(torch.uint8).to(torch.int8)


def _layer(bits: int, H: int, I: int, seed: int, scales: str):
    g = torch.Generator().manual_seed(seed)
    qmax = 7 if bits == 4 else 127
    # W1: gate rows all 1.0, up rows one-hot in K
    c1 = torch.zeros(1, 2 * I, H, dtype=torch.int32)
    c1[0, :I, :] = 1
    for n in range(I):
        c1[0, I + n, n::I] = 1
    s1 = torch.ones(1, 2 * I, 1)
    # W2: row 0 all 1.0; other rows random codes, scales over many binades
    c2 = torch.randint(-qmax - 1, qmax + 1, (1, H, I), generator=g, dtype=torch.int32)
    c2[0, 0, :] = 1
    # "tiny": down to 2^-100; "huge": 2^103 .. 2^111, where the in-register
    # dequant leaves its fast half-precision trick for the plain conversion
    # (every such chunk); either way every q*s and a*q*s stays a normal fp32
    # number, so the expected products below are exact
    lo_exp, hi_exp = {"normal": (-30, 6), "tiny": (-100, 6), "huge": (103, 111)}[scales]
    s2 = (2.0 ** torch.randint(lo_exp, hi_exp, (1, H, 1), generator=g).float()) * (1 + torch.rand(1, H, 1, generator=g))
    s2[0, 0, 0] = 1.0
    w1 = QuantResult(q=_codes(c1, bits), scale=s1, bits=bits, group_size=-1, packed=bits == 4,
                     logical_shape=(1, 2 * I, H))
    w2 = QuantResult(q=_codes(c2, bits), scale=s2, bits=bits, group_size=-1, packed=bits == 4,
                     logical_shape=(1, H, I))
    return w1, w2


def _to(r: QuantResult, dev) -> QuantResult:
    return QuantResult(q=r.q.to(dev), scale=r.scale.to(dev), bits=r.bits, group_size=r.group_size,
                       packed=r.packed, logical_shape=r.logical_shape)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("T", [16, 32, 200])
@pytest.mark.parametrize("scales", ["normal", "tiny", "huge"])
def test_exact_layer_reproduces_standalone_dequant(dev, bits, T, scales):
    """T=16 runs the streaming GEMMs, T=32 and 200 the wide ones."""
    H, I = 512, 512
    w1, w2 = (_to(r, dev) for r in _layer(bits, H, I, seed=T + bits, scales=scales))
    x = torch.eye(H, dtype=torch.bfloat16)[:T].to(dev)
    ids = torch.zeros(T, 1, dtype=torch.int32, device=dev)
    w = torch.ones(T, 1, device=dev)
    out = fused_moe_packed(x, w1, w2, ids, w).cpu()

    a = out[:, 0].float()  # the activation value, identical for every token
    silu1 = torch.nn.functional.silu(torch.tensor(1.0)).bfloat16().float()
    assert torch.all(a == silu1), "act(g=1, u=1) must be bf16(silu(1))"
    deq2 = dequantize_tensor(w2.q, w2.scale, bits, -1, torch.bfloat16, packed=bits == 4).float().cpu()[0]
    n_of_t = torch.arange(T) % I
    expected = (a[:, None] * deq2[:, n_of_t].T).bfloat16()  # bf16 x bf16 is exact in fp32
    mismatch = (out.view(torch.int16) != expected.view(torch.int16)).sum().item()
    assert mismatch == 0, f"{mismatch} of {out.numel()} outputs differ"
