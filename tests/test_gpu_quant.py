"""GPU parity of packing, unpacking, dequantization and the quantizer.

Everything here is integer or byte work, or a float computation the reference
performs with a fixed IEEE operation sequence, so the bar is bit-exactness
against the CPU oracle (oracle/lq_oracle.c) and against the golden vectors
the reference itself produced (tests/golden/).
"""

from __future__ import annotations

import glob
import hashlib
import os

import numpy as np
import pytest
import torch

from conftest import bits_u16
from llada_quant_amd.algorithms.symmetric import (
    dequantize_tensor,
    pack_int4,
    quantize_tensor,
    search_group_scale,
    unpack_int4,
)
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
DT = {torch.float32: O.F32, torch.float16: O.F16, torch.bfloat16: O.BF16}


def _np_in(w: torch.Tensor):
    """(array, dtype code) as the oracle takes it."""
    if w.dtype == torch.float32:
        return w.cpu().numpy(), O.F32
    return bits_u16(w), DT[w.dtype]


def test_unpack_every_byte_matches_the_oracle(dev):
    every = torch.arange(-128, 128, dtype=torch.int8).reshape(1, 256)
    got = unpack_int4(every.to(dev)).cpu().numpy()
    assert np.array_equal(got, O.unpack_int4(every.numpy()))


def test_pack_every_pair_roundtrips(dev):
    v = torch.arange(-8, 8, dtype=torch.int8)
    pairs = torch.stack(torch.meshgrid(v, v, indexing="ij"), -1).reshape(1, -1).to(dev)
    packed = pack_int4(pairs)
    assert np.array_equal(packed.cpu().numpy(), O.pack_int4(pairs.cpu().numpy()))
    assert torch.equal(unpack_int4(packed), pairs)


def test_pack_nibble_order_and_range_errors(dev):
    p = pack_int4(torch.tensor([[1, 2]], dtype=torch.int8, device=dev))
    assert int(p[0, 0]) & 0x0F == 1 and (int(p[0, 0]) >> 4) & 0x0F == 2
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        pack_int4(torch.tensor([[8, 0]], dtype=torch.int8, device=dev))
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        pack_int4(torch.tensor([[-9, 0]], dtype=torch.int8, device=dev))
    with pytest.raises(ValueError, match="even"):
        pack_int4(torch.zeros(1, 3, dtype=torch.int8, device=dev))


def test_unpack_large_random_matches_the_oracle(dev):
    g = torch.Generator().manual_seed(5)
    x = torch.randint(-128, 128, (64, 2048, 512), generator=g, dtype=torch.int8)
    got = unpack_int4(x.to(dev)).cpu().numpy()
    assert np.array_equal(got, O.unpack_int4(x.numpy()))


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [16, 32, 64, 128, -1, 48])
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_dequant_bit_exact(dev, bits, group, out_dtype):
    g = torch.Generator().manual_seed(bits * 1000 + group)
    k = 256
    w = (torch.randn(3, 40, k, generator=g) * 0.02).to(torch.bfloat16)
    wn, code = _np_in(w)
    q, s, gs = O.quantize(wn, bits, group, "amax", w_dtype=code)
    out_code = DT[out_dtype]
    ref = O.dequant(q, s, bits, gs, k, out_dtype=out_code)
    got = dequantize_tensor(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), bits, gs,
                            dtype=out_dtype, packed=bits == 4)
    got_np = got.cpu().numpy() if out_dtype == torch.float32 else bits_u16(got)
    assert got_np.dtype == ref.dtype and np.array_equal(got_np, ref)


def test_dequant_odd_shapes_take_the_generic_kernel(dev):
    g = torch.Generator().manual_seed(3)
    w = torch.randn(5, 7, 50, generator=g)
    q, s, gs = O.quantize(w.numpy(), 8, 33, "amax")  # 33 does not divide 50: one group per row
    assert gs == -1
    ref = O.dequant(q, s, 8, gs, 50, out_dtype=O.BF16)
    got = dequantize_tensor(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), 8, gs, dtype=torch.bfloat16)
    assert np.array_equal(bits_u16(got), ref)


def test_dequant_large_c5_shaped_tensor(dev):
    """A full C3/C4/C5 w1 ([64, 2048, 2048] INT4, G=128) dequantizes bit-exactly."""
    g = torch.Generator().manual_seed(11)
    q = torch.randint(-128, 128, (64, 2048, 1024), generator=g, dtype=torch.int8)
    s = torch.rand(64, 2048, 16, generator=g) * 1e-2
    got = dequantize_tensor(q.to(dev), s.to(dev), 4, 128, dtype=torch.bfloat16, packed=True)
    # check a deterministic sample of rows against the oracle (full CPU dequant is slow)
    rows = np.random.default_rng(0).choice(64 * 2048, 512, replace=False)
    qn = q.reshape(-1, 1024).numpy()[rows]
    sn = s.reshape(-1, 16).numpy()[rows]
    ref = O.dequant(qn, sn, 4, 128, 2048, out_dtype=O.BF16)
    assert np.array_equal(bits_u16(got.reshape(-1, 2048)[torch.from_numpy(rows).to(dev)]), ref)


def test_dequant_without_packed_flag_fails_loudly(dev):
    q = quantize_tensor(torch.randn(2, 4, 32, device=dev), bits=4, group_size=16)
    with pytest.raises(RuntimeError):
        dequantize_tensor(q.q, q.scale, 4, 16, packed=False)
    assert dequantize_tensor(q.q, q.scale, 4, 16, packed=True).shape == (2, 4, 32)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("group", [16, 32, 64, 128, -1, 48])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("search", ["amax", "mse"])
def test_quantize_bit_exact_against_the_oracle(dev, bits, group, wdtype, search):
    g = torch.Generator().manual_seed(7 * bits + group)
    w = (torch.randn(2, 24, 192, generator=g) * 0.02).to(wdtype)
    w[0, 0, :32] = 0  # a zero group
    wn, code = _np_in(w)
    q_ref, s_ref, gs_ref = O.quantize(wn, bits, group, search, grid=16, w_dtype=code)
    res = quantize_tensor(w.to(dev), bits=bits, group_size=group, scale_search=search, search_grid=16)
    assert res.group_size == gs_ref
    assert np.array_equal(res.q.cpu().numpy(), q_ref)
    assert np.array_equal(res.scale.cpu().numpy(), s_ref)


@pytest.mark.parametrize("sdtype", [torch.bfloat16, torch.float16])
def test_quantize_with_reduced_precision_scales(dev, sdtype):
    g = torch.Generator().manual_seed(1)
    w = (torch.randn(4, 16, 256, generator=g) * 0.02).to(torch.bfloat16)
    q_ref, s_ref, _ = O.quantize(bits_u16(w), 4, 64, "mse", grid=8, w_dtype=O.BF16, scale_dtype=DT[sdtype])
    res = quantize_tensor(w.to(dev), bits=4, group_size=64, scale_dtype=sdtype, scale_search="mse", search_grid=8)
    assert res.scale.dtype == sdtype
    assert np.array_equal(res.q.cpu().numpy(), q_ref)
    assert np.array_equal(bits_u16(res.scale), s_ref)


def test_quantize_int4_unpacked_storage(dev):
    w = torch.randn(3, 8, 64, device=dev)
    a = quantize_tensor(w, bits=4, group_size=32, pack=False)
    b = quantize_tensor(w, bits=4, group_size=32, pack=True)
    assert not a.packed and a.q.shape == (3, 8, 64)
    assert torch.equal(pack_int4(a.q), b.q)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "mse_*.npz"))))
def test_quantize_matches_reference_golden_vectors(dev, path):
    z = np.load(path)
    if "q_sha256" in z.files:
        pytest.skip("hash fixture: covered by test_quantize_c5_layer_matches_reference_hash")
    code = int(z["w_dtype"])
    raw = torch.from_numpy(z["w_bits"].view(np.int16) if code != O.F32 else z["w_bits"])
    w = raw if code == O.F32 else raw.view(torch.float16 if code == O.F16 else torch.bfloat16)
    res = quantize_tensor(w.to(dev), bits=int(z["bits"]), group_size=int(z["group_size"]), scale_search="mse",
                          search_grid=int(z["grid"]))
    assert np.array_equal(res.q.cpu().numpy(), z["q"])
    assert np.array_equal(res.scale.cpu().numpy(), z["scale"])
    assert res.group_size == int(z["result_group_size"])
    assert np.array_equal(bits_u16(res.dequantize(torch.bfloat16)), z["dequant_bf16"])


@pytest.mark.parametrize("which", ["w2", "w1"])
def test_quantize_c5_layer_matches_reference_hash(dev, which):
    """A C5 w2 ([64, 2048, 1024]) and w1 ([64, 2048, 2048]), bf16 ~N(0, 0.02), INT4 G=128,
    MSE grid 16: the GPU quantizer gives the reference quantizer's exact bytes."""
    z = np.load(os.path.join(GOLDEN, f"mse_c5_{which}_layer_hash.npz"))
    gen = torch.Generator().manual_seed(int(z["seed"]))
    w = (torch.randn(*z["shape"].tolist(), generator=gen) * float(z["std"])).to(torch.bfloat16)
    res = quantize_tensor(w.to(dev), bits=4, group_size=128, scale_search="mse", search_grid=int(z["grid"]))
    assert np.array_equal(res.scale.reshape(-1)[:4096].cpu().numpy(), z["scale_head"])
    assert hashlib.sha256(res.scale.cpu().numpy().tobytes()).digest() == z["scale_sha256"].tobytes()
    assert hashlib.sha256(res.q.cpu().numpy().tobytes()).digest() == z["q_sha256"].tobytes()


def test_search_group_scale_matches_oracle_and_is_shape_preserving(dev):
    g = torch.Generator().manual_seed(2)
    w = torch.distributions.StudentT(3.0).sample((32, 512)) * 0.01
    w_g = w.reshape(32, 4, 128)
    got = search_group_scale(w_g.to(dev), bits=4, grid=8)
    assert got.shape == (32, 4, 1)
    ref = O.search_group_scale(w_g.numpy(), 4, grid=8)
    assert np.array_equal(got.cpu().numpy(), ref)
    # chunking is a no-op by construction
    assert torch.equal(search_group_scale(w_g.to(dev), bits=4, grid=8, chunk_elements=1024), got)


def test_quantizer_is_deterministic(dev):
    w = (torch.randn(64, 256, 512, device=dev) * 0.02).to(torch.bfloat16)
    a = quantize_tensor(w, bits=4, group_size=128, scale_search="mse", search_grid=16)
    b = quantize_tensor(w, bits=4, group_size=128, scale_search="mse", search_grid=16)
    assert torch.equal(a.q, b.q) and torch.equal(a.scale, b.scale)


def test_zero_tensor_quantizes_to_zero(dev):
    for search in ("amax", "mse"):
        q = quantize_tensor(torch.zeros(4, 8, 16, device=dev), bits=8, group_size=8, scale_search=search)
        assert torch.all(q.q == 0) and torch.all(q.scale == 0)


@pytest.mark.parametrize("bits,group", [(4, 128), (8, 128), (4, 32)])
def test_mse_search_extreme_magnitudes_match_the_oracle(dev, bits, group):
    """The MSE search divides by each candidate scale through its reciprocal (Markstein's
    correctly rounded quotient), falling back to the IEEE division where that does not
    apply.  Groups here span 2^-149 .. 2^120 in magnitude, with subnormal weights, zeros
    and subnormal scales: codes and scales must equal the oracle's (IEEE division) bit
    for bit."""
    rng = np.random.default_rng(bits + group)
    rows, K = 96, 256
    mag = np.exp2(rng.integers(-149, 121, size=(rows * K // group, 1))).astype(np.float64)
    w = (rng.standard_normal((rows * K // group, group)) * mag).reshape(rows, K)
    w[rng.random(w.shape) < 0.05] = 0.0
    w[::7, :group] = 0.0  # whole zero groups
    w = np.clip(w, -3e38, 3e38).astype(np.float32)
    wt = torch.from_numpy(w).to(dev)
    res = quantize_tensor(wt, bits=bits, group_size=group, scale_search="mse", search_grid=16)
    oq, os_, _ = O.quantize(w, bits, group, "mse", grid=16, w_dtype=O.F32)
    assert np.array_equal(res.scale.cpu().numpy(), os_)
    assert np.array_equal(res.q.cpu().numpy(), oq)


@pytest.mark.parametrize("bits,grid", [(4, 16), (8, 16), (4, 80)])
def test_mse_search_quotients_near_half_integers_match_the_oracle(dev, bits, grid):
    """Weights within 3 ulps of (m + 1/2) times one of the group's candidate scales: the
    MSE search's quotient shortcut must hand those to the IEEE division, and still agree
    with the oracle bit for bit.  Grid 80 also takes the candidate ratios past step 63,
    which the kernel computes per step instead of reading them from a lane."""
    rng = np.random.default_rng(11 * bits + grid)
    qmax = 2 ** (bits - 1) - 1
    groups, group = 384, 128
    amax = rng.uniform(0.01, 0.05, size=groups).astype(np.float32)
    amax_s = amax / np.float32(qmax)  # fp32 quotient, as the search forms it
    steps = rng.integers(0, grid, size=(groups, group))
    ratio = (1.0 - 0.5 * steps / grid).astype(np.float32)
    cand = amax_s[:, None] * ratio  # fp32 products: the candidate scales
    m = rng.integers(-qmax, qmax, size=(groups, group))  # |m + 1/2| <= qmax - 1/2 keeps |w| < amax
    near = ((m + 0.5) * cand.astype(np.float64)).astype(np.float32)
    w = (near.view(np.int32) + rng.integers(-3, 4, size=near.shape).astype(np.int32)).view(np.float32)
    w[:, 0] = amax * np.where(rng.random(groups) < 0.5, -1, 1).astype(np.float32)
    w = w.reshape(groups // 4, 4 * group)
    res = quantize_tensor(torch.from_numpy(w).to(dev), bits=bits, group_size=group, scale_search="mse",
                          search_grid=grid)
    oq, os_, _ = O.quantize(w, bits, group, "mse", grid=grid, w_dtype=O.F32)
    assert np.array_equal(res.scale.cpu().numpy(), os_)
    assert np.array_equal(res.q.cpu().numpy(), oq)
