"""Write reference-produced quantized checkpoints for the interop tests.

Runs LLaDA_Quant v0.2.0 itself (this build container only; the GPU box never
sees the reference): its test model (tests/unit/conftest.py TinyMoEModel,
torch.manual_seed(0)) is quantized with ``quantize_model`` and saved with
``save_quantized_checkpoint`` exactly as tests/unit/test_checkpoint_format.py
does, into ``tests/golden/ckpt_<case>/``.  Beside each artifact,
``expected.npz`` holds what the reference's ``block.w1`` / ``block.w2`` return
after quantization: the SHA-256 of their BF16 bytes and the first 64 values as
uint16 bit patterns, per layer.

    python tests/golden/make_ckpt_golden.py /root/reference
"""

from __future__ import annotations

import hashlib
import os
import shutil
import sys

import numpy as np

CASES = {
    # name: (bits, group_size, execution_mode)
    "int4_packed_g64": (4, 64, "packed"),
    "int8_reference_g64": (8, 64, "reference"),
    "int8_packed_g48": (8, 48, "packed"),  # 48 does not divide K=128: one scale per row
}


def main(ref_root: str) -> None:
    sys.path.insert(0, os.path.join(ref_root, "src"))
    sys.path.insert(0, os.path.join(ref_root, "tests", "unit"))
    import torch
    from LLaDA_Quant import QuantConfig, QuantizationManifest, quantize_model, save_quantized_checkpoint
    from conftest import TinyMoEModel

    here = os.path.dirname(os.path.abspath(__file__))
    for name, (bits, group, mode) in CASES.items():
        out = os.path.join(here, f"ckpt_{name}")
        shutil.rmtree(out, ignore_errors=True)
        torch.manual_seed(0)
        model = TinyMoEModel()
        config = QuantConfig(bits=bits, group_size=group, targets=("expert",), execution_mode=mode)
        result = quantize_model(model, config)
        manifest = QuantizationManifest(source_checkpoint="hf://test/model", config=config, targets=result.targets)
        save_quantized_checkpoint(model, manifest, out)
        expect = {}
        for i, layer in enumerate(model.layers):
            for w in ("w1", "w2"):
                bits16 = getattr(layer.mlp, w).detach().contiguous().view(torch.int16).numpy().view(np.uint16)
                expect[f"layer{i}_{w}_sha256"] = np.frombuffer(hashlib.sha256(bits16.tobytes()).digest(), np.uint8)
                expect[f"layer{i}_{w}_head"] = bits16.reshape(-1)[:64].copy()
                expect[f"layer{i}_{w}_shape"] = np.array(bits16.shape, np.int64)
        np.savez(os.path.join(out, "expected.npz"), **expect)
        print("wrote", out, sorted(os.listdir(out)))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
