"""Shared test setup.

GPU tests carry ``@pytest.mark.gpu`` and run only on a ROCm device; they never
skip themselves when no GPU is present (``-m "not gpu"`` deselects them).

The toy models below have the module tree of an LLaDA-MoE decoder stack at
toy size -- ``embed_tokens``, ``layers.<i>.mlp`` (a router ``gate`` and the
fused ``w1 [E, 2I, H]`` / ``w2 [E, H, I]`` expert weights, BF16 ~ N(0, 0.02)),
``layers.<i>.q_proj``, ``layers.<i>.input_layernorm``, ``router`` and
``lm_head`` -- so their state-dict names are those of the checkpoints the
reference writes for its test model, and only the ``mlp`` blocks are
quantization targets.
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


def _bf16_normal(shape, gen, std=0.02):
    return (torch.randn(*shape, generator=gen) * std).to(torch.bfloat16)


class ExpertMLP(nn.Module):
    """A fused expert block: router ``gate`` plus ``w1`` (gate and up rows) and ``w2``."""

    def __init__(self, num_experts=NUM_EXPERTS, hidden=HIDDEN, intermediate=INTERMEDIATE, seed=0):
        super().__init__()
        gen = torch.Generator().manual_seed(seed)
        self.gate = nn.Linear(hidden, num_experts, bias=False, dtype=torch.bfloat16)
        self.w1 = nn.Parameter(_bf16_normal((num_experts, 2 * intermediate, hidden), gen))
        self.w2 = nn.Parameter(_bf16_normal((num_experts, hidden, intermediate), gen))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Every expert on every token, averaged (fp32 on the CPU): exercises w1/w2 reads."""
        w1 = self.w1.float().cpu()
        w2 = self.w2.float().cpu()
        xs = x.float().cpu()
        half = w2.shape[-1]
        outs = []
        for e in range(w1.shape[0]):
            h = xs @ w1[e].T
            outs.append((F.silu(h[:, :half]) * h[:, half:]) @ w2[e].T)
        return torch.stack(outs).mean(0)


def _decoder_layer(index: int, seed: int) -> nn.Module:
    layer = nn.Module()
    layer.mlp = ExpertMLP(seed=seed + index)
    layer.q_proj = nn.Linear(HIDDEN, HIDDEN, bias=False, dtype=torch.bfloat16)
    layer.input_layernorm = nn.LayerNorm(HIDDEN, dtype=torch.bfloat16)
    return layer


class ToyMoE(nn.Module):
    """``layers`` decoder layers with expert MLPs, plus the modules that are never quantized."""

    def __init__(self, layers=2, seed=0):
        super().__init__()
        self.embed_tokens = nn.Embedding(VOCAB, HIDDEN)
        self.layers = nn.ModuleList(_decoder_layer(i, seed) for i in range(layers))
        self.router = nn.Linear(HIDDEN, NUM_EXPERTS, bias=False, dtype=torch.bfloat16)
        self.lm_head = nn.Linear(HIDDEN, VOCAB, bias=False, dtype=torch.bfloat16)


@pytest.fixture
def dev() -> torch.device:
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    return torch.device("cuda", 0)


@pytest.fixture
def expert_block(dev) -> ExpertMLP:
    return ExpertMLP().to(dev)


@pytest.fixture
def moe_model(dev) -> ToyMoE:
    torch.manual_seed(0)
    return ToyMoE().to(dev)


def bits_u16(t: torch.Tensor):
    """bf16/f16 tensor -> numpy uint16 bit patterns (on the CPU)."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view("uint16")
