"""Pin the CPU oracle (oracle/lq_oracle.c) before any GPU result is compared with it.

Each check is chosen so that a plausible slip in the oracle -- a swapped
nibble, a dropped sign extension, the wrong rounding mode, a transposed
gate/up split, a wrong summation order -- fails here, on the CPU:

* reference golden vectors (tests/golden/mse_*.npz, written by running the
  reference's own ``quantize_tensor`` in this container) for the MSE search;
* exhaustive brute force for pack/unpack (all 256 bytes, all 256 pairs) and
  the reference's nibble-order known answer (tests/unit/test_int4.py:45-49);
* closed forms evaluated independently with numpy's IEEE float32 arithmetic
  for amax scales, quantization and dequantization;
* torch itself for the summation order (``x.sum()`` on the CPU), routing
  (``softmax(fp32).topk``), and the permutation (stable argsort + bincount);
* an independent numpy restatement of the MoE layer for the fused op order.
"""

from __future__ import annotations

import glob
import hashlib
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def bits_to_f32(bits: np.ndarray, code: int) -> np.ndarray:
    if code == O.F32:
        return bits.astype(np.float32)
    if code == O.BF16:
        return O.bf16_bits_to_f32(bits)
    return bits.view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------
# golden vectors from the reference quantizer
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "mse_*_grid*.npz"))),
                         ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_quantizer_matches_reference_golden_vectors(path):
    d = np.load(path)
    w = d["w_bits"]
    code = int(d["w_dtype"])
    q, scale, g = O.quantize(w, bits=int(d["bits"]), group_size=int(d["group_size"]), scale_search="mse",
                             grid=int(d["grid"]), w_dtype=code)
    assert np.array_equal(q, d["q"])
    assert np.array_equal(scale.view(np.uint32), d["scale"].view(np.uint32))
    assert g == int(d["result_group_size"])
    k = w.shape[-1]
    deq = O.dequant(q, scale, int(d["bits"]), g, k)
    assert np.array_equal(deq, d["dequant_bf16"])


def test_oracle_scale_head_of_c5_layer_matches_reference():
    """First 4096 group scales of the reference's C5-sized w2 (seeded [64, 2048, 1024] bf16)."""
    d = np.load(os.path.join(GOLDEN, "mse_c5_w2_layer_hash.npz"))
    gen = torch.Generator().manual_seed(int(d["seed"]))
    shape = tuple(int(s) for s in d["shape"])
    w = (torch.randn(*shape, generator=gen) * float(d["std"])).to(torch.bfloat16)
    rows = 4096 // (shape[-1] // int(d["group_size"]))
    head = bf16_bits(w.reshape(-1, shape[-1])[:rows])
    _, scale, _ = O.quantize(head, bits=int(d["bits"]), group_size=int(d["group_size"]), scale_search="mse",
                             grid=int(d["grid"]), w_dtype=O.BF16)
    assert np.array_equal(scale.reshape(-1).view(np.uint32), d["scale_head"].view(np.uint32))


@pytest.mark.slow
def test_oracle_full_c5_layer_matches_reference_hash():
    """All 16.8M groups of the C5-sized w2: SHA-256 of codes and scales equal the reference's."""
    d = np.load(os.path.join(GOLDEN, "mse_c5_w2_layer_hash.npz"))
    gen = torch.Generator().manual_seed(int(d["seed"]))
    shape = tuple(int(s) for s in d["shape"])
    w = bf16_bits((torch.randn(*shape, generator=gen) * float(d["std"])).to(torch.bfloat16))
    q, scale, _ = O.quantize(w, bits=4, group_size=128, scale_search="mse", grid=int(d["grid"]), w_dtype=O.BF16)
    assert hashlib.sha256(q.tobytes()).digest() == d["q_sha256"].tobytes()
    assert hashlib.sha256(scale.tobytes()).digest() == d["scale_sha256"].tobytes()


# ---------------------------------------------------------------------------
# pack / unpack: brute force and known answers (symmetric.py:296-346)
# ---------------------------------------------------------------------------


def _decode_byte(b: int):
    lo, hi = b & 0xF, (b >> 4) & 0xF
    return (lo - 16 if lo >= 8 else lo), (hi - 16 if hi >= 8 else hi)


def test_unpack_every_byte_brute_force():
    allb = np.arange(256, dtype=np.uint8).view(np.int8).reshape(1, 256)
    out = O.unpack_int4(allb)
    want = np.array([v for b in range(256) for v in _decode_byte(b)], np.int8).reshape(1, 512)
    assert np.array_equal(out, want)


def test_pack_every_pair_brute_force_and_roundtrip():
    pairs = np.array([(lo, hi) for lo in range(-8, 8) for hi in range(-8, 8)], np.int8).reshape(1, -1)
    packed = O.pack_int4(pairs)
    want = np.array([(lo & 0xF) | ((hi & 0xF) << 4) for lo in range(-8, 8) for hi in range(-8, 8)],
                    np.uint8).view(np.int8).reshape(1, -1)
    assert np.array_equal(packed, want)
    assert np.array_equal(O.unpack_int4(packed), pairs)


def test_nibble_order_known_answer():
    """The reference's KAT: [1, 2] packs to one byte with low nibble 1, high nibble 2."""
    packed = O.pack_int4(np.array([[1, 2]], np.int8))
    assert packed.view(np.uint8)[0, 0] == 0x21


def test_pack_rejects_out_of_range_and_odd_shapes():
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        O.pack_int4(np.array([[8, 0]], np.int8))
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        O.pack_int4(np.array([[0, -9]], np.int8))
    with pytest.raises(ValueError, match="even"):
        O.pack_int4(np.zeros((2, 3), np.int8))


# ---------------------------------------------------------------------------
# amax quantizer and dequant: closed forms (symmetric.py:117-119, 207-293)
# ---------------------------------------------------------------------------


def _numpy_amax_quantize(wf: np.ndarray, bits: int, g: int):
    """Independent closed form with numpy float32 IEEE ops: s = amax/Qmax, q = clamp(rint(w/s))."""
    qmax = np.float32(2 ** (bits - 1) - 1)
    qmin = np.float32(-(2 ** (bits - 1)))
    wg = wf.reshape(*wf.shape[:-1], wf.shape[-1] // g, g)
    s = (np.abs(wg).max(axis=-1, keepdims=True) / qmax).astype(np.float32)
    safe = np.where(s > 0, s, np.float32(1))
    q = np.clip(np.rint(wg / safe), qmin, qmax).astype(np.int8)
    return q.reshape(wf.shape), s[..., 0]


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("g", [32, 64, 128])
@pytest.mark.parametrize("code", [O.F32, O.BF16, O.F16])
def test_amax_quantize_closed_form(bits, g, code):
    rng = np.random.default_rng(bits * 1000 + g + code)
    wf = (rng.standard_normal((6, 3, 256)) * 0.02).astype(np.float32)
    if code == O.BF16:
        wbits = O.f32_to_bf16_bits(wf)
    elif code == O.F16:
        wbits = wf.astype(np.float16).view(np.uint16)
    else:
        wbits = wf
    wf = bits_to_f32(wbits, code)
    q, s, geff = O.quantize(wbits, bits=bits, group_size=g, scale_search="amax", w_dtype=code)
    wq, ws = _numpy_amax_quantize(wf, bits, g)
    assert geff == g
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))
    if bits == 4:
        q = O.unpack_int4(q)
    assert np.array_equal(q, wq)
    # invariants of the reference tests: |err| <= s/2 and the amax element maps to +-Qmax
    deq = bits_to_f32(O.dequant(O.pack_int4(q) if bits == 4 else q, s, bits, g, 256), O.BF16)
    err = np.abs(deq.astype(np.float64) - wf.astype(np.float64)).reshape(6, 3, 256 // g, g)
    bound = s[..., None].astype(np.float64) / 2 + np.abs(deq).reshape(err.shape) * 2.0 ** -8
    assert (err <= bound + 1e-12).all()
    qmax = 2 ** (bits - 1) - 1
    assert (np.abs(q.reshape(6, 3, 256 // g, g)).max(axis=-1) == qmax).all()


def test_zero_tensor_gives_zero_scale_and_codes():
    q, s, _ = O.quantize(np.zeros((4, 256), np.float32), bits=4, group_size=128, scale_search="mse", grid=16)
    assert not q.any() and not s.any()
    q, s, _ = O.quantize(np.zeros((4, 256), np.float32), bits=8, group_size=128, scale_search="amax")
    assert not q.any() and not s.any()


def test_qmax_known_answers():
    # int8: the amax element of a group maps to 127 with s = amax / 127 exactly
    w = np.zeros((1, 128), np.float32)
    w[0, 5] = -2.54
    q, s, _ = O.quantize(w, bits=8, group_size=128)
    assert s[0, 0] == np.float32(np.float32(2.54) / np.float32(127))
    assert q[0, 5] == -127
    q, s, _ = O.quantize(w, bits=4, group_size=128)
    assert s[0, 0] == np.float32(np.float32(2.54) / np.float32(7))
    assert O.unpack_int4(q)[0, 5] == -7


def test_per_row_fallback_when_group_does_not_divide():
    """G=48 does not divide K=96*... -> one group per row, group_size recorded as -1."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((5, 100)) * 0.1).astype(np.float32)
    q, s, g = O.quantize(w, bits=8, group_size=48)
    assert g == -1 and s.shape == (5, 1)
    wq, ws = _numpy_amax_quantize(w, 8, 100)
    assert np.array_equal(q, wq) and np.array_equal(s, ws)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("out_code", [O.BF16, O.F32, O.F16])
def test_dequant_closed_form(bits, out_code):
    rng = np.random.default_rng(7 + bits)
    q8 = rng.integers(-(2 ** (bits - 1)), 2 ** (bits - 1), size=(9, 256), dtype=np.int8)
    s = (rng.random((9, 4)) * 0.01 + 1e-4).astype(np.float32)
    prod = (q8.reshape(9, 4, 64).astype(np.float32) * s[..., None]).reshape(9, 256)
    want = {O.BF16: O.f32_to_bf16_bits(prod), O.F32: prod, O.F16: prod.astype(np.float16).view(np.uint16)}[out_code]
    got = O.dequant(O.pack_int4(q8) if bits == 4 else q8, s, bits, 64, 256, out_dtype=out_code)
    assert np.array_equal(got, want)


def test_bf16_rounding_known_answers():
    # half-way cases round to even (NaN is left out: torch's vectorized CPU cast and its
    # scalar cast disagree on the NaN payload, and no finite dequant input produces one)
    vals = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -0.0, np.inf, 3.0e38, 1.0e-40], np.float32)
    got = O.f32_to_bf16_bits(vals)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert got[0] == 0x3F80 and got[1] == 0x3F82


# ---------------------------------------------------------------------------
# MSE search: torch's CPU summation order and search invariants
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("n", list(range(1, 300)) + [511, 512, 513, 1000, 1024, 2048, 4095, 4096, 8191, 8192])
def test_torch_cpu_sum_order_is_bit_exact(n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) ** 2 * 10.0 ** rng.uniform(-6, 2, n)).astype(np.float32)
    want = torch.from_numpy(x).sum().item()
    assert np.float32(O.torch_cpu_sum(x)).view(np.uint32) == np.float32(want).view(np.uint32)


def _group_sse(w: np.ndarray, s: np.ndarray, bits: int) -> np.ndarray:
    qmax, qmin = 2 ** (bits - 1) - 1, -(2 ** (bits - 1))
    safe = np.where(s > 0, s, 1.0).astype(np.float64)
    q = np.clip(np.rint(w / safe), qmin, qmax)
    return ((q * safe - w) ** 2).sum(axis=-1)


@pytest.mark.parametrize("bits", [4, 8])
def test_mse_search_invariants(bits):
    rng = np.random.default_rng(11)
    w = (rng.standard_t(3, size=(64, 4, 128)) * 0.01).astype(np.float32)
    s = O.search_group_scale(w, bits=bits, grid=24)
    amax = (np.abs(w).max(axis=-1, keepdims=True) / np.float32(2 ** (bits - 1) - 1)).astype(np.float32)
    assert (s > 0).all() and (s <= amax).all()
    sse_mse = _group_sse(w.astype(np.float64), s.astype(np.float64), bits)
    sse_amax = _group_sse(w.astype(np.float64), amax.astype(np.float64), bits)
    assert (sse_mse <= sse_amax * (1 + 1e-5)).all()
    if bits == 4:
        assert sse_mse.sum() < 0.95 * sse_amax.sum()  # the reference's >5% gain on Student-t(3)
    # grid=1 has the single candidate ratio 1.0: the amax scale
    assert np.array_equal(O.search_group_scale(w, bits=bits, grid=1), amax)


def test_mse_candidate_ratios_are_the_python_double_rounded_to_fp32():
    """With one nonzero element per group, every candidate gives the same error class; the
    winner must be one of base * fp32(1 - 0.5 * step / grid) for some step."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((32, 1, 64)) * 0.05).astype(np.float32)
    s = O.search_group_scale(w, bits=4, grid=24)[..., 0]
    base = (np.abs(w).max(axis=-1) / np.float32(7)).astype(np.float32)
    cands = np.stack([base * np.float32(1.0 - 0.5 * st / 24) for st in range(24)], -1)
    assert (cands == s[..., None]).any(axis=-1).all()


# ---------------------------------------------------------------------------
# routing, permutation, MoE layer
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("T,E,k,renorm", [(300, 16, 2, True), (512, 64, 8, False), (64, 64, 8, True),
                                          (50, 128, 4, False)])
def test_routing_matches_torch_softmax_topk(T, E, k, renorm):
    g = torch.Generator().manual_seed(T + E)
    logits = torch.randn(T, E, generator=g)
    ids, w = O.route_topk(logits.numpy(), k, renorm)
    probs = F.softmax(logits, dim=-1, dtype=torch.float32)
    tv, ti = probs.topk(k, dim=-1)
    if renorm:
        tv = tv / tv.sum(dim=-1, keepdim=True)
    assert np.array_equal(ids, ti.numpy().astype(np.int32))
    np.testing.assert_allclose(w, tv.numpy(), rtol=2e-6, atol=1e-9)


def test_routing_ties_go_to_the_lower_expert():
    logits = np.zeros((3, 8), np.float32)
    logits[1, 5] = 1.0
    ids, _ = O.route_topk(logits, 3, False)
    assert ids.tolist() == [[0, 1, 2], [5, 0, 1], [0, 1, 2]]


@pytest.mark.parametrize("T,k,E", [(64, 8, 64), (4096, 8, 64), (256, 2, 16), (7, 3, 5), (1, 1, 1)])
def test_permutation_is_a_stable_argsort(T, k, E):
    rng = np.random.default_rng(T)
    ids = rng.integers(0, E, size=(T, k)).astype(np.int32)
    counts, offsets, sorted_ = O.moe_permute(ids, E)
    flat = ids.reshape(-1)
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
    assert np.array_equal(sorted_, np.argsort(flat, kind="stable"))


def test_expert_token_stats_known_answer():
    """tests/unit/test_moe_regime.py:89-97: counts [3, 2, 1, 0]."""
    counts, offsets, sorted_ = O.moe_permute(np.array([[0, 1], [0, 2], [0, 1]], np.int32), 4)
    assert counts.tolist() == [3, 2, 1, 0]
    assert offsets.tolist() == [0, 3, 5, 6, 6]
    assert sorted_.tolist() == [0, 2, 4, 1, 5, 3]


def _numpy_moe(x, w1, w2, ids, wts):
    """Independent restatement: per (token, slot) fp64 products with the reference's roundings."""
    bf = lambda a: O.bf16_bits_to_f32(O.f32_to_bf16_bits(np.asarray(a, np.float32)))  # noqa: E731
    I = w2.shape[-1]
    out = np.zeros((x.shape[0], w2.shape[1]), np.float64)
    for t in range(x.shape[0]):
        for j in range(ids.shape[1]):
            e = ids[t, j]
            h = w1[e].astype(np.float64) @ x[t].astype(np.float64)
            gb, ub = bf(h[:I]), bf(h[I:])
            act = bf(bf(gb.astype(np.float64) / (1.0 + np.exp(-gb.astype(np.float64)))) * ub)
            out[t] += wts[t, j] * (w2[e].astype(np.float64) @ act.astype(np.float64))
    return out


def test_moe_forward_matches_independent_restatement():
    E, H, I, T, k = 4, 128, 64, 9, 2
    rng = np.random.default_rng(0)
    x = O.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    w1 = O.f32_to_bf16_bits((rng.standard_normal((E, 2 * I, H)) * 0.02).astype(np.float32))
    w2 = O.f32_to_bf16_bits((rng.standard_normal((E, H, I)) * 0.02).astype(np.float32))
    ids, wts = O.route_topk(rng.standard_normal((T, E)).astype(np.float32), k, True)
    got = O.moe_forward(x, w1, w2, ids, wts)
    want = _numpy_moe(O.bf16_bits_to_f32(x), O.bf16_bits_to_f32(w1), O.bf16_bits_to_f32(w2), ids, wts)
    scale = np.abs(want).max()
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-3 * scale)
    # a gate/up swap is caught: the swapped layer differs by far more than the tolerance
    swapped = np.concatenate([w1[:, I:], w1[:, :I]], axis=1)
    assert np.abs(O.moe_forward(x, swapped, w2, ids, wts) - want).max() > 0.2 * scale


def test_torch_reference_layer_agrees_with_the_oracle():
    """oracle/torch_ref.packed_layer (the timed CPU baseline) computes the same layer."""
    from oracle import torch_ref

    E, H, I, T, k = 4, 256, 128, 16, 2
    g = torch.Generator().manual_seed(2)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).float()
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).float()
    q1, s1, _ = O.quantize(w1.numpy(), bits=4, group_size=128)
    q2, s2, _ = O.quantize(w2.numpy(), bits=4, group_size=128)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g)
    out, ids = torch_ref.packed_layer(x, logits, torch.from_numpy(q1), torch.from_numpy(s1), torch.from_numpy(q2),
                                      torch.from_numpy(s2), 4, 128, k, renormalize=True)
    oids, ow = O.route_topk(logits.numpy(), k, True)
    assert np.array_equal(ids.numpy(), oids)
    ref = O.moe_forward(bf16_bits(x), O.dequant(q1, s1, 4, 128, H), O.dequant(q2, s2, 4, 128, I), oids, ow)
    diff = np.abs(out.float().numpy() - ref)
    assert diff.max() < 2e-2 and diff.sum() / np.abs(ref).sum() < 5e-3


# ---------------------------------------------------------------------------
# the MoE forward against the reference's own executable restatements
# ---------------------------------------------------------------------------

def _moe_golden_cases():
    import sys

    sys.path.insert(0, GOLDEN)
    import moe_inputs

    return moe_inputs


@pytest.mark.parametrize("case", [c[0] for c in _moe_golden_cases().CASES])
def test_moe_forward_matches_reference_expert_forward(case):
    """oq_moe_forward against the reference's expert_forward (benchmarks/bench_numerical.py:28-36)
    and FusedExpertBlock.forward (tests/unit/conftest.py:37-43), both executed by
    tests/golden/make_moe_golden.py on the reference-quantized weights.  Those are dense over
    every expert and averaged, so the oracle runs with every token routed to all E experts at
    weight 1/E.  They accumulate gate, up and act in fp32 where fused_moe rounds each to bf16,
    so the match is to the north-star tolerance (max-abs 2e-2, mean-relative 5e-3), which a
    swapped gate/up split, a missing SwiGLU factor or a transposed down projection all exceed.
    The oracle's quantize + dequant must first reproduce the reference's dequantized bytes."""
    mi = _moe_golden_cases()
    name, E, H, I, T, bits, group, search, grid, seed = next(c for c in mi.CASES if c[0] == case)
    z = np.load(os.path.join(GOLDEN, f"moe_{name}.npz"))
    w1b, w2b, xb = mi.case_inputs(E, H, I, T, seed)
    deq = []
    for wb, k, key in ((w1b, H, "d1_sha256"), (w2b, I, "d2_sha256")):
        q, s, g = O.quantize(wb, bits=bits, group_size=group, scale_search=search, grid=grid, w_dtype=O.BF16)
        d = O.dequant(q, s, bits, g, k)
        assert hashlib.sha256(d.astype(np.uint16).tobytes()).digest() == z[key].tobytes(), key
        deq.append(d)
    d1, d2 = deq
    ids = np.tile(np.arange(E, dtype=np.int32), (T, 1))
    wts = np.full((T, E), 1.0 / E, np.float32)
    got = O.moe_forward(xb, d1, d2, ids, wts).astype(np.float64)

    def close(ref):
        diff = np.abs(got - ref)
        return diff.max() < 2e-2 and diff.sum() / np.abs(ref).sum() < 5e-3

    ref = z["expert_forward"].astype(np.float64)
    assert close(ref), (np.abs(got - ref).max(), np.abs(got - ref).sum() / np.abs(ref).sum())
    assert close(z["fused_block_forward"].astype(np.float64))
    # planted slips the check must catch
    swapped = np.concatenate([d1[:, I:], d1[:, :I]], axis=1)
    assert not close(O.moe_forward(xb, swapped, d2, ids, wts).astype(np.float64))
    d2t = np.ascontiguousarray(d2.reshape(E, H, I)[:, ::-1, :])  # rows of W2 in the wrong order
    assert not close(O.moe_forward(xb, d1, d2t, ids, wts).astype(np.float64))
