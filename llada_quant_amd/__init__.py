"""llada_quant_amd: LLaDA_Quant's quantized MoE expert path, native on MI355X (gfx950).

Packed groupwise-symmetric INT4/INT8 expert weights are consumed directly by
hand-written HIP kernels (``liblladaq.so``, a C-ABI library loaded through
ctypes): a top-k softmax router, a stable expert permutation, grouped
W4A16/W8A16 GEMMs with in-register bit-exact dequantization, fused SwiGLU and
top-k combine, a bit-exact dequant kernel and a GPU MSE quantizer.

The surface is the reference's: ``QuantConfig``, ``ExecutionMode.PACKED``,
``quantize_model``, the ``block.w1`` property,
``fused_moe(x, w1, w2, gating_output, topk_ids)`` and the checkpoint format
(``save_quantized_checkpoint`` / ``load_quantized_weights``, which reads the
packed buffers straight into GPU memory).
"""

from .api import QuantizationResult, TargetingError, quantize_model, quantized_model
from .config import ExecutionMode, QuantConfig
from .formats.manifest import QuantizationManifest
from .formats.safetensors import load_quantized_weights, save_quantized_checkpoint
from .runtime.fused_moe import fused_moe, fused_moe_packed, moe_layer
from .runtime.moe import PackedExpertTensor
from .runtime.routing import expert_token_stats, moe_permute, route_topk

__version__ = "0.1.0"

__all__ = [
    "QuantConfig",
    "ExecutionMode",
    "QuantizationResult",
    "QuantizationManifest",
    "TargetingError",
    "save_quantized_checkpoint",
    "load_quantized_weights",
    "quantize_model",
    "quantized_model",
    "fused_moe",
    "fused_moe_packed",
    "moe_layer",
    "PackedExpertTensor",
    "route_topk",
    "moe_permute",
    "expert_token_stats",
    "__version__",
]
