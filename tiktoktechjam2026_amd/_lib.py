"""ctypes binding of the in-tree C-ABI library ``libmpk.so`` (declared in ``include/mpk.h``).

The library is loaded lazily on first use and must already be built
(``python -m tiktoktechjam2026_amd.build`` or ``__graft_entry__.build()``).
There is no fallback: a missing library or a non-zero status raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch

from .build import LIB_PATH

F32 = 0
F16 = 1

MPK_OK = 0
MPK_EINVAL = 1001
MPK_EUNSUPPORTED = 1002
MPK_EALIGN = 1003

_c_void_p = ctypes.c_void_p
_c_int = ctypes.c_int
_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_float = ctypes.c_float
_c_i64_p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); mirrors include/mpk.h
SIGNATURES = {
    "mpk_version": (_c_int, []),
    "mpk_status_string": (ctypes.c_char_p, [_c_int]),
    "mpk_device_synchronize": (_c_int, []),
    "mpk_layernorm": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i32, _c_float, _c_void_p],
    ),
    "mpk_linear": (
        _c_int,
        [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_i64, _c_i32, _c_i32, _c_int, _c_void_p],
    ),
    "mpk_linear_auto_variant": (_c_int, [_c_i64, _c_i32, _c_i32]),
    "mpk_linear_qscaled": (
        _c_int,
        [
            _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i32, _c_i32, _c_i32, _c_float,
            _c_int, _c_void_p,
        ],
    ),
    "mpk_linear_residual": (
        _c_int,
        [_c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i32, _c_i32, _c_int, _c_void_p],
    ),
    "mpk_linear_residual_layernorm": (
        _c_int,
        [
            _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
            _c_int, _c_i64, _c_i32, _c_float, _c_int, _c_void_p,
        ],
    ),
    "mpk_linear_residual_layernorm_auto_variant": (_c_int, [_c_i64, _c_i32]),
    "mpk_linear_add_layernorm": (
        _c_int,
        [
            _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
            _c_int, _c_i64, _c_i32, _c_i32, _c_float, _c_void_p,
        ],
    ),
    "mpk_ffn_residual_layernorm": (
        _c_int,
        [
            _c_void_p, _c_int, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
            _c_void_p, _c_void_p, _c_int, _c_i64, _c_i32, _c_i32, _c_float, _c_int, _c_void_p,
        ],
    ),
    "mpk_ffn_residual_layernorm_auto_variant": (_c_int, [_c_i64, _c_i32, _c_i32]),
    "mpk_causal_attention": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_int, _c_i64_p, _c_i64_p, _c_i64_p, _c_i64_p,
            _c_i32, _c_i32, _c_i32, _c_i32, _c_float, _c_int, _c_void_p, _c_int, _c_void_p,
        ],
    ),
    "mpk_attention_auto_variant": (_c_int, [_c_i32, _c_i32, _c_i32, _c_i32]),
    "mpk_causal_attention_prescaled": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64_p, _c_i64_p, _c_i64_p, _c_i64_p,
            _c_i32, _c_i32, _c_i32, _c_i32, _c_int, _c_void_p, _c_int, _c_void_p,
        ],
    ),
    "mpk_layer_tail": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i32,
            _c_i32, _c_float, _c_float, _c_int, _c_void_p,
        ],
    ),
    "mpk_layer_tail_supported": (_c_int, [_c_i32, _c_i32]),
    "mpk_layer_tail_qscaled": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i32,
            _c_i32, _c_float, _c_float, _c_float, _c_int, _c_void_p,
        ],
    ),
    "mpk_attention_layer_tail": (
        _c_int,
        [
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
            _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_int, _c_i64, _c_i32,
            _c_i32, _c_i32, _c_i32, _c_float, _c_int, _c_float, _c_float, _c_void_p,
        ],
    ),
    "mpk_attention_layer_tail_supported": (_c_int, [_c_i32, _c_i32, _c_i32]),
    "mpk_attention_layer_tail_rows": (_c_i32, []),
    "mpk_layernorm_qkv": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i32, _c_float, _c_int, _c_void_p],
    ),
    "mpk_layernorm_qkv_supported": (_c_int, [_c_i32]),
    "mpk_layernorm_qkv_qscaled": (
        _c_int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_i64, _c_i32, _c_float, _c_float, _c_int,
         _c_void_p],
    ),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load ``libmpk.so`` once and attach the C signatures; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP kernels first "
                    "(python -m tiktoktechjam2026_amd.build)"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != MPK_OK:
        message = load().mpk_status_string(int(status)).decode()
        raise RuntimeError(f"{what} failed with status {status}: {message}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return F32
    if dtype == torch.float16:
        return F16
    raise ValueError(f"unsupported dtype {dtype}")


def stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def strides4(values) -> ctypes.Array:
    return (ctypes.c_int64 * 4)(*[int(v) for v in values])
