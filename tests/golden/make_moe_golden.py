"""Write reference-executed golden vectors for the expert forward.

The oracle's MoE forward (oracle/lq_oracle.c oq_moe_forward) restates the
gate / up split, the SwiGLU and the down projection of the external
fused_moe.  This script runs the reference's own executable restatements of
that contract on the inputs of moe_inputs.CASES:

  * benchmarks/bench_numerical.py:28-36 ``expert_forward`` -- a dense fp32
    pass over every expert, averaged over the experts;
  * tests/unit/conftest.py:37-43 ``FusedExpertBlock.forward`` -- the same
    with einsum, mean over the experts;

each over the weights the reference quantizer produces and dequantizes
(algorithms/symmetric.py: quantize_tensor, then QuantResult.dequantize to
bf16).  It stores the SHA-256 of the dequantized bf16 bytes and both fp32
outputs; the inputs are regenerated from moe_inputs (integer arithmetic only).

Run in the build container only (the reference tree does not exist on the
GPU box):

    python tests/golden/make_moe_golden.py [/root/reference]
"""

from __future__ import annotations

import hashlib
import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import moe_inputs  # noqa: E402


def _load(path: str, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16)


def main(root: str) -> None:
    sys.path.insert(0, os.path.join(root, "src"))
    from LLaDA_Quant.algorithms.symmetric import quantize_tensor  # noqa: E402

    bench = _load(os.path.join(root, "benchmarks", "bench_numerical.py"), "ref_bench_numerical")
    conftest = _load(os.path.join(root, "tests", "unit", "conftest.py"), "ref_conftest")
    for name, E, H, I, T, bits, group, search, grid, seed in moe_inputs.CASES:
        w1b, w2b, xb = moe_inputs.case_inputs(E, H, I, T, seed)
        w1, w2, x = _bf16(w1b), _bf16(w2b), _bf16(xb)
        q1 = quantize_tensor(w1, bits=bits, group_size=group, scale_search=search, search_grid=grid)
        q2 = quantize_tensor(w2, bits=bits, group_size=group, scale_search=search, search_grid=grid)
        d1, d2 = q1.dequantize(torch.bfloat16), q2.dequantize(torch.bfloat16)
        out = bench.expert_forward(d1, d2, x.float())
        block = conftest.FusedExpertBlock(num_experts=E, hidden=H, intermediate=I)
        with torch.no_grad():
            block.w1.data = d1.clone()
            block.w2.data = d2.clone()
            out_block = block(x)
        sha = lambda t: np.frombuffer(hashlib.sha256(t.contiguous().view(torch.int16).numpy().tobytes()).digest(),
                                      np.uint8)
        np.savez_compressed(
            os.path.join(HERE, f"moe_{name}.npz"),
            experts=np.int32(E), hidden=np.int32(H), intermediate=np.int32(I), tokens=np.int32(T),
            bits=np.int32(bits), group_size=np.int32(group), scale_search=np.array(search), grid=np.int32(grid),
            seed=np.int64(seed),
            d1_sha256=sha(d1), d2_sha256=sha(d2),
            expert_forward=out.numpy().astype(np.float32),
            fused_block_forward=out_block.float().numpy().astype(np.float32),
        )
        print("wrote", name, "out", tuple(out.shape), float(out.abs().mean()))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
