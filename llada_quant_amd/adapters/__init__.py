"""Model integration: structural detection and quantization of fused expert blocks."""

from .llada_moe import (  # noqa: F401
    describe_fused_expert_block,
    find_expert_blocks,
    is_fused_expert_block,
    quantize_llada_experts,
    restore_llada_experts_from_buffers,
)
