"""Symmetric groupwise INT8 / packed-INT4 quantization, computed by HIP kernels.

Drop-in for ``LLaDA_Quant.algorithms.symmetric`` (v0.2.0,
``src/LLaDA_Quant/algorithms/symmetric.py``): same functions, arguments,
results and error messages, but every tensor computation runs in
``liblladaq.so`` on the GPU.  The numerical contract is the reference's,
bit for bit:

* groups of ``group_size`` run along the last (K) axis; when ``group_size``
  is -1 or does not divide K, each row is one group (the reference's
  "per-tensor" fallback, symmetric.py:85-90, 252-256);
* ``scale = amax / Qmax`` (fp32 IEEE divide), or the MSE clip search over
  ``search_grid`` ratios in ``[1 - max_shrink, 1]`` whose per-group squared
  error is summed in torch's CPU order (symmetric.py:122-204);
* ``q = clamp(round_half_even(w / safe), Qmin, Qmax)`` as int8; at 4 bits two
  values share a byte, element 2i in the low nibble (symmetric.py:296-313);
* ``dequantize = cast(fp32(q) * fp32(scale))`` (symmetric.py:272-293).

Argument validation runs on the host before any device work, so the same
``ValueError``s are raised for CPU tensors; the computation itself requires
HIP tensors and raises otherwise.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from ..runtime import _lib

SCALE_SEARCH_AMAX = "amax"
SCALE_SEARCH_MSE = "mse"
KNOWN_SCALE_SEARCH = (SCALE_SEARCH_AMAX, SCALE_SEARCH_MSE)


def qmax_for_bits(bits: int) -> int:
    """Largest code of a signed symmetric ``bits``-bit quantizer (symmetric.py:29-31)."""
    return (1 << (bits - 1)) - 1


def qmin_for_bits(bits: int) -> int:
    """Most negative code, ``-Qmax - 1`` (symmetric.py:34-36)."""
    return -(1 << (bits - 1))


@dataclass
class QuantResult:
    """Integer codes plus per-group scales (symmetric.py:39-82).

    ``q`` is always int8; when ``packed`` it holds two 4-bit codes per byte and
    its last dimension is half of ``logical_shape``'s.  ``scale`` has shape
    ``logical_shape[:-1] + (num_groups,)``; ``group_size`` is -1 for the
    one-group-per-row fallback.
    """

    q: torch.Tensor
    scale: torch.Tensor
    bits: int
    group_size: int
    packed: bool = False
    logical_shape: Tuple[int, ...] = ()

    def __post_init__(self) -> None:
        if not self.logical_shape:
            shape = list(self.q.shape)
            if self.packed:
                shape[-1] *= 2
            self.logical_shape = tuple(shape)

    def dequantize(self, dtype: torch.dtype = torch.float32) -> torch.Tensor:
        return dequantize_tensor(self.q, self.scale, self.bits, self.group_size, dtype=dtype,
                                 packed=self.packed)

    def storage_bytes(self) -> int:
        """Bytes of codes plus scales actually held."""
        return self.q.numel() * self.q.element_size() + self.scale.numel() * self.scale.element_size()


def _as_groups(w: torch.Tensor, group_size: int) -> Tuple[torch.Tensor, int]:
    """View ``[..., K]`` as ``[..., K/G, G]``; one group per row when G does not fit."""
    k = w.shape[-1]
    if group_size == -1 or k % group_size != 0:
        return w, 1
    return w.reshape(*w.shape[:-1], k // group_size, group_size), k // group_size


def _effective_group(k: int, group_size: int) -> int:
    return k if (group_size == -1 or group_size <= 0 or k % group_size != 0) else group_size


def validate_int4_layout(shape: Sequence[int], group_size: int) -> None:
    """Raise unless a byte-aligned int4 packing exists (symmetric.py:93-108)."""
    if shape[-1] % 2 != 0:
        raise ValueError(
            f"int4 packing needs an even last dimension, got {tuple(shape)}; "
            "the last axis is the K axis and two values share one byte"
        )
    if group_size != -1 and group_size % 2 != 0:
        raise ValueError(
            f"int4 packing needs an even group_size so groups stay byte-aligned, got {group_size}"
        )


def _float_input(w: torch.Tensor) -> torch.Tensor:
    # the reference upcasts anything that is not f16/bf16/f32 to f32 first
    if w.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        w = w.to(torch.float32)
    return w.contiguous()


def search_group_scale(
    w_g: torch.Tensor,
    bits: int,
    grid: int = 24,
    max_shrink: float = 0.5,
    chunk_elements: int = 64_000_000,
) -> torch.Tensor:
    """MSE-optimal clip scale per group of ``w_g`` ``[..., num_groups, G]``.

    Tries ratios ``1 - max_shrink * step / grid`` (step = 0..grid-1) of the
    amax scale and keeps, per group, the first one with the strictly smallest
    squared reconstruction error; zero groups get 0 (symmetric.py:122-204).
    One kernel launch covers every group: the GPU kernel holds a group in
    registers, so ``chunk_elements`` (the reference's memory bound) is accepted
    for compatibility and changes nothing, exactly like chunking in the
    reference.  Returns fp32 scales shaped ``[..., num_groups, 1]``.
    """
    if grid < 1:
        raise ValueError(f"grid must be >= 1, got {grid}")
    if not 0.0 <= max_shrink < 1.0:
        raise ValueError(f"max_shrink must lie in [0, 1), got {max_shrink}")
    if bits not in (8, 4):
        raise ValueError(f"bits must be 8 or 4, got {bits}")
    w = _float_input(w_g)
    device = _lib.require_hip(w)
    glen = w.shape[-1] if w.dim() else 1
    n_groups = w.numel() // max(glen, 1)
    out = torch.empty(*w.shape[:-1], 1, dtype=torch.float32, device=device)
    if n_groups:
        lib = _lib.load()
        with torch.cuda.device(device):
            rc = lib.lq_search_group_scale(_lib.ptr(w), _lib.dtype_code(w.dtype, "weights"), n_groups, glen, bits,
                                           grid, float(max_shrink), _lib.ptr(out), _lib.stream(device))
        _lib.check(rc, "search_group_scale")
    return out


def quantize_tensor(
    w: torch.Tensor,
    bits: int = 8,
    group_size: int = 128,
    scale_dtype: torch.dtype = torch.float32,
    pack: bool = True,
    scale_search: str = SCALE_SEARCH_AMAX,
    search_grid: int = 24,
) -> QuantResult:
    """Quantize ``w`` per group along its last axis (symmetric.py:207-269).

    One kernel computes the scales (amax, or the MSE search), the codes and,
    for ``bits=4, pack=True``, the nibble packing.  ``pack=False`` at 4 bits
    keeps one code per byte.
    """
    if bits not in (8, 4):
        raise ValueError(f"bits must be 8 or 4, got {bits}")
    if w.numel() == 0:
        raise ValueError("cannot quantize an empty tensor")
    if bits == 4 and pack:
        validate_int4_layout(w.shape, group_size)
    if scale_search not in KNOWN_SCALE_SEARCH:
        raise ValueError(
            f"scale_search must be one of {list(KNOWN_SCALE_SEARCH)}, got {scale_search!r}"
        )
    if search_grid < 1 and scale_search == SCALE_SEARCH_MSE:
        raise ValueError(f"grid must be >= 1, got {search_grid}")
    s_code = _lib.dtype_code(scale_dtype, "scale_dtype")
    w = _float_input(w)
    device = _lib.require_hip(w)

    logical_shape = tuple(w.shape)
    k = logical_shape[-1]
    rows = w.numel() // k
    g = _effective_group(k, group_size)
    num_groups = k // g
    packed = bits == 4 and pack
    q = torch.empty(*logical_shape[:-1], k // 2 if packed else k, dtype=torch.int8, device=device)
    scale = torch.empty(*logical_shape[:-1], num_groups, dtype=scale_dtype, device=device)
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.lq_quantize(
            _lib.ptr(w), _lib.dtype_code(w.dtype, "weights"), rows, k, bits, int(packed), group_size,
            _lib.LQ_SCALE_MSE if scale_search == SCALE_SEARCH_MSE else _lib.LQ_SCALE_AMAX,
            int(search_grid), 0.5, _lib.ptr(q), _lib.ptr(scale), s_code, _lib.stream(device),
        )
    _lib.check(rc, "quantize_tensor")
    return QuantResult(
        q=q,
        scale=scale,
        bits=bits,
        group_size=group_size if num_groups > 1 else -1,
        packed=packed,
        logical_shape=logical_shape,
    )


def dequantize_tensor(
    q: torch.Tensor,
    scale: torch.Tensor,
    bits: int,
    group_size: int,
    dtype: torch.dtype = torch.float32,
    packed: bool = False,
) -> torch.Tensor:
    """``cast(fp32(q) * fp32(scale))`` with the grouping of ``quantize_tensor``.

    Bit-exact to the reference (symmetric.py:272-293).  Passing packed codes
    without ``packed=True`` (or scales of the wrong shape) raises instead of
    returning a plausible tensor, as the reference's reshape does.
    """
    if bits not in (8, 4):
        raise ValueError(f"bits must be 8 or 4, got {bits}")
    if packed and q.dtype != torch.int8:
        raise ValueError(f"packed int4 storage must be int8, got {q.dtype}")
    if q.dtype != torch.int8:
        q = q.to(torch.int8)
    k = q.shape[-1] * (2 if packed else 1)
    rows = q.numel() // max(q.shape[-1], 1) if q.dim() else 1
    g = _effective_group(k, group_size)
    ng = k // g if k else 1
    if scale.numel() != rows * ng:
        raise RuntimeError(
            f"scale of shape {tuple(scale.shape)} does not match codes {tuple(q.shape)} "
            f"(bits={bits}, group_size={group_size}, packed={packed}): expected {rows * ng} scales"
        )
    device = _lib.require_hip(q, scale)
    out_dtype = dtype if dtype in _lib.DTYPE_CODES else torch.float32
    out = torch.empty(*q.shape[:-1], k, dtype=out_dtype, device=device)
    if out.numel():
        s = scale.contiguous()
        if s.dtype not in _lib.DTYPE_CODES:
            s = s.to(torch.float32)
        lib = _lib.load()
        with torch.cuda.device(device):
            rc = lib.lq_dequant(_lib.ptr(q.contiguous()), _lib.ptr(s), _lib.dtype_code(s.dtype, "scale"), rows, k,
                                4 if packed else 8, group_size, _lib.ptr(out),
                                _lib.dtype_code(out_dtype, "dtype"), _lib.stream(device))
        _lib.check(rc, "dequantize_tensor")
    return out if out_dtype == dtype else out.to(dtype)


def pack_int4(q8: torch.Tensor) -> torch.Tensor:
    """Two int4 codes per byte along the last axis (symmetric.py:296-313)."""
    if q8.shape[-1] % 2 != 0:
        raise ValueError("last dim must be even for int4 packing")
    out_shape = (*q8.shape[:-1], q8.shape[-1] // 2)
    if q8.numel() == 0:
        return torch.empty(out_shape, dtype=torch.int8, device=q8.device)
    device = _lib.require_hip(q8)
    src = q8
    if src.dtype != torch.int8:
        lo, hi = int(src.min()), int(src.max())
        if hi > 7 or lo < -8:
            raise ValueError(f"int4 packing needs values in [-8, 7], got [{lo}, {hi}]")
        src = src.to(torch.int8)
    src = src.contiguous()
    out = torch.empty(out_shape, dtype=torch.int8, device=device)
    flag = torch.zeros(1, dtype=torch.int32, device=device)
    rows = src.numel() // src.shape[-1]
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.lq_pack_int4(_lib.ptr(src), rows, src.shape[-1], _lib.ptr(out), _lib.ptr(flag),
                              _lib.stream(device))
    _lib.check(rc, "pack_int4")
    if int(flag.item()) != 0:
        raise ValueError(f"int4 packing needs values in [-8, 7], got [{int(src.min())}, {int(src.max())}]")
    return out


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of :func:`pack_int4`, sign-extending both nibbles (symmetric.py:316-346)."""
    if packed.dtype != torch.int8:
        raise ValueError(f"packed int4 storage must be int8, got {packed.dtype}")
    out = torch.empty(*packed.shape[:-1], packed.shape[-1] * 2, dtype=torch.int8, device=packed.device)
    if packed.numel() == 0:
        return out
    device = _lib.require_hip(packed)
    src = packed.contiguous()
    rows = src.numel() // src.shape[-1]
    lib = _lib.load()
    with torch.cuda.device(device):
        rc = lib.lq_unpack_int4(_lib.ptr(src), rows, src.shape[-1], _lib.ptr(out), _lib.stream(device))
    _lib.check(rc, "unpack_int4")
    return out


def storage_bytes(numel: int, bits: int, group_size: int, scale_bytes: int = 4) -> int:
    """Bytes of ``numel`` weights stored at ``bits`` with per-group scales (symmetric.py:349-362)."""
    if bits == 8:
        value_bytes = numel
    elif bits == 4:
        value_bytes = numel // 2
    else:
        raise ValueError(f"bits must be 8 or 4, got {bits}")
    groups = 1 if group_size == -1 else max(1, numel // group_size)
    return value_bytes + groups * scale_bytes


def block_k_is_scale_aligned(block_k: int, group_size: int) -> bool:
    """True when a K tile of ``block_k`` never straddles a scale group (symmetric.py:365-378)."""
    if group_size == -1:
        return True
    if block_k <= 0 or group_size <= 0:
        return False
    return block_k % group_size == 0 or group_size % block_k == 0


def validate_block_k_alignment(block_k: int, group_size: int) -> None:
    """Raise unless ``block_k`` addresses whole scale groups (symmetric.py:381-394)."""
    if not block_k_is_scale_aligned(block_k, group_size):
        raise ValueError(
            f"BLOCK_SIZE_K={block_k} cannot address group_size={group_size} scales "
            "exactly: one must divide the other, or a K-tile straddles a group "
            "boundary and half of it is dequantized with the wrong scale"
        )


def aligned_block_k_values(group_size: int, candidates: Sequence[int]) -> list:
    """The tile sizes of ``candidates`` that address groups exactly (symmetric.py:397-399)."""
    return [k for k in candidates if block_k_is_scale_aligned(k, group_size)]


__all__ = [
    "SCALE_SEARCH_AMAX",
    "SCALE_SEARCH_MSE",
    "KNOWN_SCALE_SEARCH",
    "QuantResult",
    "qmax_for_bits",
    "qmin_for_bits",
    "validate_int4_layout",
    "search_group_scale",
    "quantize_tensor",
    "dequantize_tensor",
    "pack_int4",
    "unpack_int4",
    "storage_bytes",
    "block_k_is_scale_aligned",
    "validate_block_k_alignment",
    "aligned_block_k_values",
]
