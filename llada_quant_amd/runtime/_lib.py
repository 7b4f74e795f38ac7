"""ctypes binding of ``liblladaq.so``, the HIP (gfx950) C-ABI library.

Every compute entry point of the package goes through here.  There is no CPU
or eager-torch fallback: if the library is missing, or a tensor is not on a
HIP device, the call raises.  torch is imported first so that the library's
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch already
loaded (one runtime, one set of streams).
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "liblladaq.so")

LQ_OK, LQ_ERR_VALUE, LQ_ERR_UNSUPPORTED, LQ_ERR_RUNTIME = 0, 1, 2, 3
LQ_F32, LQ_F16, LQ_BF16 = 0, 1, 2
LQ_SCALE_AMAX, LQ_SCALE_MSE = 0, 1
ABI_VERSION = 3
LQ_MOE_FOLDED_SCALES = 1
LQ_MOE_GENERAL_KERNEL = 2
LQ_MOE_WIDE_KERNEL = 4
LQ_MOE_STREAM_KERNEL = 8
LQ_MOE_FUSED_LAYER = 16

DTYPE_CODES = {torch.float32: LQ_F32, torch.float16: LQ_F16, torch.bfloat16: LQ_BF16}

_P, _I64, _I32, _D, _SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/lladaq.h
SIGNATURES = {
    "lq_abi_version": (_I32, []),
    "lq_last_error": (ctypes.c_char_p, []),
    "lq_pack_int4": (_I32, [_P, _I64, _I64, _P, _P, _P]),
    "lq_unpack_int4": (_I32, [_P, _I64, _I64, _P, _P]),
    "lq_dequant": (_I32, [_P, _P, _I32, _I64, _I64, _I32, _I64, _P, _I32, _P]),
    "lq_quantize": (_I32, [_P, _I32, _I64, _I64, _I32, _I32, _I64, _I32, _I32, _D, _P, _P, _I32, _P]),
    "lq_search_group_scale": (_I32, [_P, _I32, _I64, _I64, _I32, _I32, _D, _P, _P]),
    "lq_route_topk": (_I32, [_P, _I32, _I64, _I32, _I32, _I32, _P, _P, _P]),
    "lq_gather_topk_weights": (_I32, [_P, _P, _I32, _I64, _I32, _I32, _I32, _P, _P, _P]),
    "lq_moe_permute": (_I32, [_P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "lq_moe_workspace_bytes": (_SZ, [_I64, _I32, _I32, _I32, _I32]),
    "lq_moe_forward": (_I32, [_P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _I32, _I64, _I64, _I32, _P, _P,
                              _P, _SZ, _P, _P]),
    "lq_moe_layer": (_I32, [_P, _P, _I32, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _I32, _I64, _I64,
                            _I32, _P, _SZ, _P, _P, _P]),
    "lq_moe_layer_noalloc": (_I32, [_P, _P, _I32, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _I32, _I64,
                                    _I64, _I32, _P, _P, _P]),
    "lq_moe_profile_events": (_I32, [_P, _I32]),
    "lq_moe_sync_bytes": (_SZ, []),
    "lq_moe_workspace_init": (_I32, [_P, _P]),
    "lq_moe_status": (_I32, [_P, _P, _I32, _P]),
    "lq_quant_linear": (_I32, [_P, _I64, _I32, _I32, _P, _P, _I32, _I64, _I32, _P, _SZ, _P, _P]),
    "lq_linear_workspace_bytes": (_SZ, [_I64, _I32, _I32]),
    "lq_route_gemm_topk": (_I32, [_P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P]),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load and type the library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built. Build the HIP library first: "
                "python -m llada_quant_amd.build"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        version = lib.lq_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"liblladaq.so ABI version {version}, expected {ABI_VERSION}; rebuild it")
        _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Raise the reference's exception type for a non-zero LQ_* status."""
    if rc == LQ_OK:
        return
    msg = load().lq_last_error().decode("utf-8", "replace")
    if rc == LQ_ERR_VALUE:
        raise ValueError(msg)
    if rc == LQ_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def require_hip(*tensors: torch.Tensor) -> torch.device:
    """The device every operand lives on; raises unless it is one HIP device."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                "llada_quant_amd computes on the GPU through its HIP kernels; "
                f"got a tensor on {t.device}. Move the tensors (or the model) to a ROCm device first."
            )
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"operands on different devices: {device} and {t.device}")
    if device is None:
        raise RuntimeError("no tensor operand")
    return device


def ptr(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def dtype_code(dtype: torch.dtype, what: str) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"{what} must be float32, float16 or bfloat16, got {dtype}") from None


def moe_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """A MoE workspace of at least ``nbytes`` bytes whose sync region is zero.

    The library's MoE calls need the sync region at the start of their
    workspace zero on entry and leave it zero, so a workspace allocated here
    serves any number of later calls (one stream at a time).  Only that
    region is cleared (a fill kernel, no memset node under graph capture): the
    rest is scratch every call overwrites, and a C5-sized layer's workspace
    is about 1 GB.
    """
    sync = int(load().lq_moe_sync_bytes())
    ws = torch.empty(max(int(nbytes), sync, 1), dtype=torch.uint8, device=device)
    ws[:sync].zero_()
    return ws


def check_status(workspace: torch.Tensor, what: str) -> None:
    """With ``LLADAQ_CHECK_STATUS=1``: synchronise and raise if a bounded wait of the
    kernels gave up since the last check (their output is then wrong)."""
    if os.environ.get("LLADAQ_CHECK_STATUS", "0") in ("", "0"):
        return
    st = ctypes.c_uint32(0)
    rc = load().lq_moe_status(ptr(workspace), ctypes.byref(st), 1, stream(workspace.device))
    check(rc, what)
    if st.value:
        raise RuntimeError(f"{what}: a kernel's bounded wait gave up (status 0x{st.value:x}); the output is wrong")
