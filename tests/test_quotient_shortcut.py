"""The quantizer's quotient shortcut, checked in IEEE float32 arithmetic on the CPU.

``quot_code`` in ``llada_quant_amd/csrc/lq_quant.hip`` never forms the correctly
rounded quotient RN(x / s) when it can avoid it.  With y within 1 ulp of
RN(1 / s) it takes q0 = RN(x y) and r = rint(q0), and keeps r when

    |q0 - r| < RN(0.5 - |q0| 2^-18)     and     2^-100 <= s <= 2^126,

dividing otherwise.  Its comment proves that an accepted r equals
rint(RN(x / s)), the code the reference's ``(w / scale).round_()`` gives.  These
tests check that claim with numpy's float32 operations (each correctly
rounded, ``np.rint`` rounding half to even) on inputs built to sit within a
few ulps of half-integers, where a looser test would fail, and that the test
still accepts almost every quotient of ordinary weights.
"""

from __future__ import annotations

import numpy as np

F = np.float32


def _accept(q0: np.ndarray, factor: float) -> np.ndarray:
    r = np.rint(q0)
    t = (0.5 - np.abs(q0.astype(np.float64)) * factor).astype(F)  # one rounding, as the FMA
    return np.abs(q0 - r) < t


def _adversarial(rng, n_scales: int = 4000, per_scale: int = 64):
    """Scales over [2^-100, 2^126] (mantissas random, and near 1 and 2) and weights within
    4 ulps of (m + 1/2) s, or up to 128 ulps (either side of the test's margin), for m up
    to 2^19 -- past the test's 2^18 ceiling."""
    e = rng.integers(-100, 126, size=n_scales)
    mant = rng.uniform(1.0, 2.0, size=n_scales)
    mant[::3] = 1.0 + rng.integers(0, 8, size=mant[::3].shape) * 2.0 ** -23
    mant[1::3] = 2.0 - rng.integers(1, 8, size=mant[1::3].shape) * 2.0 ** -23
    s = np.ldexp(mant, e).astype(F)
    s = s[(s >= F(2.0 ** -100)) & (s <= F(2.0 ** 126))]
    mag = np.exp2(rng.uniform(0, 19, size=(s.size, per_scale)))
    m = np.floor(mag * np.where(rng.random(mag.shape) < 0.5, -1, 1))
    with np.errstate(over="ignore"):
        near = ((m + 0.5) * s[:, None].astype(np.float64)).astype(F)
        off = np.where(rng.random(near.shape) < 0.4, rng.integers(-4, 5, size=near.shape),
                       rng.integers(-128, 129, size=near.shape))
        x = (near.view(np.int32) + off.astype(np.int32)).view(F)
    ok = np.isfinite(x)
    return np.broadcast_to(s[:, None], x.shape)[ok], x[ok]


def _reciprocals(s: np.ndarray):
    """RN(1/s) and its neighbours one ulp either side."""
    y = (F(1.0) / s).astype(F)
    return [y, np.nextafter(y, F(0.0)), np.nextafter(y, F(np.inf))]


def test_accepted_codes_equal_the_correctly_rounded_quotients_code():
    rng = np.random.default_rng(0)
    s, x = _adversarial(rng)
    with np.errstate(over="ignore", invalid="ignore"):
        truth = np.rint(x / s)
        for y in _reciprocals(s):
            q0 = x * y
            acc = _accept(q0, 2.0 ** -18)
            assert acc.sum() > 0.1 * acc.size  # the adversarial set is not all rejected
            bad = acc & (np.rint(q0) != truth)
            assert not bad.any(), (x[bad][:4], s[bad][:4])


def test_the_adversarial_inputs_catch_a_looser_acceptance():
    """With no margin (accept whenever q0 is not exactly a half-integer) or a margin of
    |q0| 2^-23, below the product's error, the same inputs give wrong codes: the set has
    the power to fail a shortcut whose margin is too small."""
    rng = np.random.default_rng(0)
    s, x = _adversarial(rng)
    with np.errstate(over="ignore", invalid="ignore"):
        truth = np.rint(x / s)
        q0 = x * _reciprocals(s)[2]
        for factor in (0.0, 2.0 ** -23):
            assert (_accept(q0, factor) & (np.rint(q0) != truth)).any()


def test_ordinary_weights_rarely_take_the_division():
    """C5-like weights: bf16 N(0, 0.02), group 128, INT4 candidates 1 - 0.5 step/16 of
    amax/7: fewer than 1 quotient in 5000 leaves the shortcut."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((2048, 128)) * 0.02).astype(F)
    amax_s = np.abs(w).max(axis=1) / F(7)
    rejected = total = 0
    with np.errstate(over="ignore", invalid="ignore"):
        for step in range(16):
            s = (amax_s * F(1.0 - 0.5 * step / 16))[:, None].astype(F)
            y = (F(1.0) / s).astype(F)
            q0 = w * y
            acc = _accept(q0, 2.0 ** -18)
            assert (np.rint(q0)[acc] == np.rint(w / s)[acc]).all()
            rejected += int((~acc).sum())
            total += acc.size
    assert rejected < total / 5000
