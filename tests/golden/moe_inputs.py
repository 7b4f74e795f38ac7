"""Deterministic bf16 inputs for the expert-forward golden vectors.

The fixtures written by make_moe_golden.py are pinned to inputs that this
module regenerates bit for bit on any machine: integer arithmetic only
(xorshift64* streams), no floating-point library call, no framework RNG.
A value is a bf16 bit pattern with a random sign, a random exponent in
[emin, emax] and a random 7-bit mantissa.
"""

from __future__ import annotations

import numpy as np

_MASK = (1 << 64) - 1


def _xorshift64star(seed: int, n: int) -> np.ndarray:
    """n uint64 draws of xorshift64* from a nonzero seed (vectorised over 64 lanes)."""
    lanes = 64
    state = np.array([((seed * 0x9E3779B97F4A7C15 + 0x632BE59BD9B4E019 * (i + 1)) & _MASK) | 1
                      for i in range(lanes)], dtype=np.uint64)
    steps = -(-n // lanes)
    out = np.empty((steps, lanes), dtype=np.uint64)
    with np.errstate(over="ignore"):
        for s in range(steps):
            state ^= state >> np.uint64(12)
            state ^= state << np.uint64(25)
            state ^= state >> np.uint64(27)
            out[s] = state * np.uint64(0x2545F4914F6CDD1D)
    return out.reshape(-1)[:n]


def bf16_bits(seed: int, shape, emin: int, emax: int) -> np.ndarray:
    """bf16 bit patterns of the given shape: sign, exponent in [emin, emax], mantissa."""
    n = int(np.prod(shape))
    r = _xorshift64star(seed, n)
    sign = (r >> np.uint64(63)).astype(np.uint16)
    exp = (emin + (r >> np.uint64(32)) % np.uint64(emax - emin + 1)).astype(np.uint16)
    mant = ((r >> np.uint64(8)) & np.uint64(0x7F)).astype(np.uint16)
    return ((sign << 15) | (exp << 7) | mant).reshape(shape)


def weights(seed: int, shape) -> np.ndarray:
    """Weight-like bf16 values, magnitudes 2^-10 .. 2^-5 (~0.001 .. 0.06)."""
    return bf16_bits(seed, shape, 117, 122)


def tokens(seed: int, shape) -> np.ndarray:
    """Activation-like bf16 values, magnitudes 2^-3 .. 2^1 (~0.13 .. 4)."""
    return bf16_bits(seed, shape, 124, 128)


# (name, experts, hidden, intermediate, tokens, bits, group, scale_search, grid, seed)
CASES = [
    ("c1_e16_h1024_i512_t16_int4_g128_amax", 16, 1024, 512, 16, 4, 128, "amax", 16, 101),
    ("e4_h128_i64_t33_int4_g64_mse16", 4, 128, 64, 33, 4, 64, "mse", 16, 202),
    ("e8_h256_i128_t24_int8_g128_mse24", 8, 256, 128, 24, 8, 128, "mse", 24, 303),
]


def case_inputs(E: int, H: int, I: int, T: int, seed: int):
    """(w1 [E, 2I, H], w2 [E, H, I], x [T, H]) as bf16 bit patterns."""
    return weights(seed, (E, 2 * I, H)), weights(seed + 1, (E, H, I)), tokens(seed + 2, (T, H))
