"""Shared test setup.

GPU tests carry ``@pytest.mark.gpu`` and run only on a ROCm device; they never
skip themselves when no GPU is present (``-m "not gpu"`` deselects them).
The fakes below mirror the reference's test fixtures
(tests/unit/conftest.py:10-76 of LLaDA_Quant v0.2.0): a fused expert block
with BF16 ``w1 [E, 2I, H]`` / ``w2 [E, H, I]`` ~ N(0, 0.02) and a two-layer
model that also holds modules that must never be quantized.
"""

from __future__ import annotations

import os
import sys

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# every MoE call in the tests reads back its workspace's status word: a
# bounded wait inside a kernel that gave up fails the test instead of passing
# wrong numbers silently
os.environ.setdefault("LLADAQ_CHECK_STATUS", "1")

HIDDEN = 128
INTERMEDIATE = 64
NUM_EXPERTS = 4
VOCAB = 32


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950) and liblladaq.so")
    config.addinivalue_line("markers", "slow: CPU check over a full configuration-sized tensor (tens of seconds)")


class FusedExpertBlock(nn.Module):
    """Fused w1/w2 layout of TritonFusedMoEBlock: w1 [E, 2I, H], w2 [E, H, I]."""

    def __init__(self, num_experts=NUM_EXPERTS, hidden=HIDDEN, intermediate=INTERMEDIATE, seed=0):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.gate = nn.Linear(hidden, num_experts, bias=False).to(torch.bfloat16)
        self.w1 = nn.Parameter((torch.randn(num_experts, 2 * intermediate, hidden, generator=gen) * 0.02)
                               .to(torch.bfloat16))
        self.w2 = nn.Parameter((torch.randn(num_experts, hidden, intermediate, generator=gen) * 0.02)
                               .to(torch.bfloat16))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Dense over all experts (fp32), enough to exercise w1/w2 access."""
        w1, w2 = self.w1.float(), self.w2.float()
        i = w2.shape[-1]
        gate = torch.einsum("th,enh->etn", x.float(), w1[:, :i])
        up = torch.einsum("th,enh->etn", x.float(), w1[:, i:])
        return torch.einsum("etk,enk->etn", F.silu(gate) * up, w2).mean(0)


class TinyMoEModel(nn.Module):
    """Two MoE layers plus pieces that must never be quantized."""

    def __init__(self, layers=2, seed=0):
        super().__init__()
        self.embed_tokens = nn.Embedding(VOCAB, HIDDEN)
        self.layers = nn.ModuleList()
        for index in range(layers):
            layer = nn.Module()
            layer.mlp = FusedExpertBlock(seed=seed + index)
            layer.q_proj = nn.Linear(HIDDEN, HIDDEN, bias=False).to(torch.bfloat16)
            layer.input_layernorm = nn.LayerNorm(HIDDEN).to(torch.bfloat16)
            self.layers.append(layer)
        self.router = nn.Linear(HIDDEN, NUM_EXPERTS, bias=False).to(torch.bfloat16)
        self.lm_head = nn.Linear(HIDDEN, VOCAB, bias=False).to(torch.bfloat16)


@pytest.fixture
def dev() -> torch.device:
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch.device("cuda", 0)


@pytest.fixture
def expert_block(dev) -> FusedExpertBlock:
    return FusedExpertBlock().to(dev)


@pytest.fixture
def moe_model(dev) -> TinyMoEModel:
    torch.manual_seed(0)
    return TinyMoEModel().to(dev)


def bits_u16(t: torch.Tensor):
    """bf16/f16 tensor -> numpy uint16 bit patterns (on the CPU)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view("uint16")
