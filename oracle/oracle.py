"""numpy front end of the CPU oracle (``liblq_oracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, always as the checker (or the
timed CPU baseline), never by the product package.

Every function restates a piece of Ahmed-Hedhili-se/LLaDA_Quant v0.2.0; the
citations are on the C functions in ``lq_oracle.c``.  Tensors are numpy
arrays; bf16/f16 data travels as ``uint16`` bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liblq_oracle.so")

F32, F16, BF16 = 0, 1, 2
_lib = None


def build() -> str:
    """Compile ``liblq_oracle.so`` with the recipe in ``oracle/Makefile``."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE, "liblq_oracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, I32, D = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double
        L.oq_f32_to_bf16.restype = ctypes.c_uint16
        L.oq_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oq_torch_cpu_sum.restype = ctypes.c_float
        L.oq_torch_cpu_sum.argtypes = [P, I64]
        L.oq_search_group_scale.argtypes = [P, I32, I64, I64, I32, I32, D, P]
        L.oq_quantize.argtypes = [P, I32, I64, I64, I32, I64, I32, I32, D, P, P, I32]
        L.oq_pack_int4.argtypes = [P, I64, I64, P]
        L.oq_unpack_int4.argtypes = [P, I64, P]
        L.oq_unpack_int4.restype = None
        L.oq_dequant.argtypes = [P, P, I32, I64, I64, I32, I64, P, I32]
        L.oq_route_topk.argtypes = [P, I32, I64, I32, I32, I32, P, P]
        L.oq_moe_permute.argtypes = [P, I64, I32, I32, P, P, P]
        L.oq_moe_forward.argtypes = [P, I64, I32, I32, I32, I32, P, P, P, P, P]
        L.oq_effective_group.restype = I64
        L.oq_effective_group.argtypes = [I64, I64]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


def _dtype_code(a: np.ndarray) -> int:
    if a.dtype == np.float32:
        return F32
    raise TypeError(f"pass f32 arrays, or uint16 bits with an explicit dtype code; got {a.dtype}")


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} failed with status {rc}")


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """torch's fp32 -> bf16 rounding (half to even; NaN -> 0x7FC0), as bits."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[np.isnan(x)] = 0x7FC0
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def torch_cpu_sum(x: np.ndarray) -> float:
    """x.sum() of one contiguous fp32 row in torch's CPU reduction order."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(lib().oq_torch_cpu_sum(_p(x), x.size))


def effective_group(k: int, group_size: int) -> int:
    return int(lib().oq_effective_group(k, group_size))


# ---------------------------------------------------------------------------
# quantizer / packing / dequant
# ---------------------------------------------------------------------------


def search_group_scale(w: np.ndarray, bits: int, grid: int = 24, max_shrink: float = 0.5,
                       w_dtype: int | None = None) -> np.ndarray:
    """Scales [..., ng, 1] for grouped weights [..., ng, G] (symmetric.py:122-204)."""
    w = np.ascontiguousarray(w)
    code = _dtype_code(w) if w_dtype is None else w_dtype
    glen = w.shape[-1]
    ng = w.size // glen
    out = np.empty(ng, np.float32)
    _check(lib().oq_search_group_scale(_p(w), code, ng, glen, bits, grid, max_shrink, _p(out)),
           "search_group_scale")
    return out.reshape(*w.shape[:-1], 1)


def quantize(w: np.ndarray, bits: int = 8, group_size: int = 128, scale_search: str = "amax",
             grid: int = 24, max_shrink: float = 0.5, w_dtype: int | None = None,
             scale_dtype: int = F32):
    """(q, scale, effective_group) per quantize_tensor (symmetric.py:207-269)."""
    w = np.ascontiguousarray(w)
    code = _dtype_code(w) if w_dtype is None else w_dtype
    k = w.shape[-1]
    rows = w.size // k
    g = effective_group(k, group_size)
    ng = k // g
    q = np.empty((*w.shape[:-1], k // 2 if bits == 4 else k), np.int8)
    scale = np.empty((*w.shape[:-1], ng), np.float32 if scale_dtype == F32 else np.uint16)
    _check(lib().oq_quantize(_p(w), code, rows, k, bits, group_size, int(scale_search == "mse"),
                             grid, max_shrink, _p(q), _p(scale), scale_dtype), "quantize")
    return q, scale, (g if ng > 1 else -1)


def pack_int4(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    k = q.shape[-1]
    out = np.empty((*q.shape[:-1], k // 2), np.int8)
    rc = lib().oq_pack_int4(_p(q), q.size // max(k, 1), k, _p(out))
    if rc == 1:
        raise ValueError("int4 packing needs values in [-8, 7]")
    if rc == 2:
        raise ValueError("last dim must be even for int4 packing")
    return out


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int8)
    out = np.empty((*packed.shape[:-1], packed.shape[-1] * 2), np.int8)
    lib().oq_unpack_int4(_p(packed), packed.size, _p(out))
    return out


def dequant(q: np.ndarray, scale: np.ndarray, bits: int, group_size: int, k: int,
            out_dtype: int = BF16, scale_dtype: int = F32) -> np.ndarray:
    """(fp32(q) * fp32(s)).to(out_dtype) (symmetric.py:272-293); bf16/f16 as uint16 bits."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    scale = np.ascontiguousarray(scale)
    rows = q.size // q.shape[-1]
    out = np.empty((*q.shape[:-1], k), np.float32 if out_dtype == F32 else np.uint16)
    _check(lib().oq_dequant(_p(q), _p(scale), scale_dtype, rows, k, bits, group_size, _p(out),
                            out_dtype), "dequant")
    return out


# ---------------------------------------------------------------------------
# routing / permutation / MoE layer
# ---------------------------------------------------------------------------


def route_topk(logits: np.ndarray, k: int, renormalize: bool, logits_dtype: int | None = None):
    logits = np.ascontiguousarray(logits)
    code = _dtype_code(logits) if logits_dtype is None else logits_dtype
    T, E = logits.shape
    ids = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.float32)
    _check(lib().oq_route_topk(_p(logits), code, T, E, k, int(renormalize), _p(ids), _p(w)),
           "route_topk")
    return ids, w


def moe_permute(ids: np.ndarray, num_experts: int):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, k = ids.shape
    counts = np.empty(num_experts, np.int32)
    offsets = np.empty(num_experts + 1, np.int32)
    sorted_ = np.empty(T * k, np.int32)
    _check(lib().oq_moe_permute(_p(ids), T, k, num_experts, _p(counts), _p(offsets), _p(sorted_)),
           "moe_permute")
    return counts, offsets, sorted_


def moe_forward(x_bits: np.ndarray, w1_bits: np.ndarray, w2_bits: np.ndarray, ids: np.ndarray,
                weights: np.ndarray) -> np.ndarray:
    """fp32 output of the dequantize-then-fused_moe layer (bf16 inputs as uint16 bits)."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    w1_bits = np.ascontiguousarray(w1_bits, dtype=np.uint16)
    w2_bits = np.ascontiguousarray(w2_bits, dtype=np.uint16)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    weights = np.ascontiguousarray(weights, dtype=np.float32)
    T, H = x_bits.shape
    E, two_i, _ = w1_bits.shape
    I = two_i // 2
    k = ids.shape[1]
    out = np.empty((T, H), np.float32)
    _check(lib().oq_moe_forward(_p(x_bits), T, H, I, E, k, _p(w1_bits), _p(w2_bits), _p(ids),
                                _p(weights), _p(out)), "moe_forward")
    return out
