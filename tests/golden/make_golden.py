"""Write the golden vectors for the reference's MSE scale search.

``search_group_scale`` (algorithms/symmetric.py:122-204) and
``quantize_tensor(scale_search="mse")`` (:207-269) are the one part of the
path that no closed form pins: which clip ratio wins a near tie depends on
torch's CPU summation order for the per-group squared error.  This script
runs the reference itself (pure Python + torch, CPU) on seeded inputs and
stores inputs and outputs as ``.npz`` fixtures next to it.

Run in the build container only (the reference tree does not exist on the
GPU box):

    python tests/golden/make_golden.py [/root/reference]          # all but the w1 hash
    python tests/golden/make_golden.py /root/reference c5w1       # the C5 w1 hash

The fixtures are data: inputs as bit patterns, outputs as the reference
returned them.  Nothing here is shipped or imported by the product.
"""

from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _bits(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16 or t.dtype == torch.float16:
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.contiguous().numpy()


def _cases():
    """(name, weight tensor, bits, group_size, grid, dtype code)."""
    g = torch.Generator().manual_seed(1234)
    bf = (torch.randn(2, 64, 256, generator=g) * 0.02).to(torch.bfloat16)
    yield "bf16_g128_int4_grid16", bf, 4, 128, 16
    yield "bf16_g128_int4_grid24", bf, 4, 128, 24
    yield "bf16_g128_int8_grid16", bf, 8, 128, 16
    yield "bf16_g64_int4_grid8", bf, 4, 64, 8
    yield "bf16_g32_int4_grid24", bf, 4, 32, 24
    heavy = (torch.distributions.StudentT(3.0).sample((32, 512)) * 0.01).float()
    yield "f32_heavy_g128_int4_grid24", heavy, 4, 128, 24
    yield "f32_heavy_g128_int8_grid24", heavy, 8, 128, 24
    # per-row fallback (48 does not divide 100): one group of 100 per row,
    # which exercises the tail of the summation order
    odd = (torch.randn(8, 16, 100, generator=g) * 0.05).to(torch.bfloat16)
    yield "bf16_fallback_k100_int4_grid16", odd, 4, 48, 16
    f16 = (torch.randn(4, 32, 128, generator=g) * 0.02).to(torch.float16)
    yield "f16_g128_int4_grid16", f16, 4, 128, 16


def c5_hash_fixture(quantize_tensor, name: str, shape, seed: int) -> None:
    """A C5-sized tensor (bf16 ~N(0, 0.02), INT4, G=128, MSE grid 16): too big to store, so
    store the seed and the SHA-256 of the reference's q and scale bytes."""
    gen = torch.Generator().manual_seed(seed)
    w = (torch.randn(*shape, generator=gen) * 0.02).to(torch.bfloat16)
    res = quantize_tensor(w, bits=4, group_size=128, scale_search="mse", search_grid=16)
    np.savez_compressed(
        os.path.join(HERE, f"mse_c5_{name}_layer_hash.npz"),
        seed=np.int64(seed),
        shape=np.array(w.shape, np.int64),
        std=np.float64(0.02),
        bits=np.int32(4),
        group_size=np.int32(128),
        grid=np.int32(16),
        q_sha256=np.frombuffer(hashlib.sha256(res.q.numpy().tobytes()).digest(), np.uint8),
        scale_sha256=np.frombuffer(hashlib.sha256(res.scale.numpy().tobytes()).digest(), np.uint8),
        scale_head=res.scale.reshape(-1)[:4096].numpy(),
    )
    print("wrote c5", name, "hash fixture")


def main(reference_root: str, only: str = "") -> None:
    sys.path.insert(0, os.path.join(reference_root, "src"))
    from LLaDA_Quant.algorithms.symmetric import quantize_tensor  # noqa: E402

    if only == "c5w1":
        # a full w1 of one C5 layer: [64, 2 * 1024, 2048] (gate and up rows)
        c5_hash_fixture(quantize_tensor, "w1", (64, 2048, 2048), 20251202)
        return

    torch.manual_seed(0)
    for name, w, bits, group, grid in _cases():
        res = quantize_tensor(w, bits=bits, group_size=group, scale_search="mse",
                              search_grid=grid)
        dtype_code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[w.dtype]
        np.savez_compressed(
            os.path.join(HERE, f"mse_{name}.npz"),
            w_bits=_bits(w),
            w_dtype=np.int32(dtype_code),
            bits=np.int32(bits),
            group_size=np.int32(group),
            grid=np.int32(grid),
            q=res.q.numpy(),
            scale=res.scale.numpy(),
            result_group_size=np.int32(res.group_size),
            dequant_bf16=_bits(res.dequantize(torch.bfloat16)),
        )
        print("wrote", name, tuple(w.shape), "q", tuple(res.q.shape), "scale", tuple(res.scale.shape))

    # one C5-sized w2 of one layer: [64, 2048, 1024]
    c5_hash_fixture(quantize_tensor, "w2", (64, 2048, 1024), 20251201)
    # and a w1 ([64, 2048, 2048]): python tests/golden/make_golden.py <root> c5w1


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference", sys.argv[2] if len(sys.argv) > 2 else "")
