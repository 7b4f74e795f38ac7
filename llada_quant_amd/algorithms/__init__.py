"""Groupwise symmetric quantization (the reference's ``algorithms`` package)."""

from .symmetric import (  # noqa: F401
    QuantResult,
    dequantize_tensor,
    pack_int4,
    qmax_for_bits,
    qmin_for_bits,
    quantize_tensor,
    search_group_scale,
    unpack_int4,
)
