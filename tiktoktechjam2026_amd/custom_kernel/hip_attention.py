"""Causal flash-attention operators backed by the gfx950 HIP kernel in ``libmpk.so``.

Mirrors the reference's ``custom_kernel/triton_attention.py``:
``is_supported`` (:235), ``is_fp16_supported`` (:249),
``launch_causal_attention`` (:264), ``causal_attention`` (:320) and
``fp16_causal_attention`` (:341).  Inputs are ``[batch, heads, seq, head_dim]``
views (typically strided views of the packed QKV projection) with a unit
head-dim stride; the output is a fresh contiguous ``[batch, seq, heads,
head_dim]`` tensor, which is the ``[tokens, d_model]`` layout the output
projection reads without a transpose.

Differences from the reference, all widening: any sequence length (the
reference accepts 128 and 1024 only), head_dim in {8, 16, 32, 64, 128, 256}, an
optional key-padding mask, and FP32 inputs handled by the same FP16-MFMA kernel.

FP32 inputs.  The reference's FP32 kernel runs its dot products in TF32 (a 10-bit
mantissa with FP32's 8-bit exponent, ``custom_kernel/triton_attention.py:85,
105-110``).  FP16 has the same 10-bit mantissa but a 5-bit exponent: normal values
span about 6.1e-5 .. 65504 only.  So the kernels first scale q (per query row), k
and v (per workgroup, over the keys it reads) by powers of two that put the largest
magnitude of each in [2^13, 2^14), round the scaled values to FP16, and undo the
scales exactly - on the score in the FP32 FMA that subtracts the running max, and on
the output.  Any finite FP32 input keeps FP16's 11-bit significand: nothing
overflows, and values down to 2^-27 of their row's (or tile's) largest keep full
precision.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from .. import _ops
from .._lib import F16, F32

HEAD_DIMS = (8, 16, 32, 64, 128, 256)


def _layout_ok(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dtype: torch.dtype) -> bool:
    """Device, dtype, shape and stride checks (what ``torch.compile`` can trace)."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return False
    if not (q.dtype == k.dtype == v.dtype == dtype):
        return False
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        return False
    if q.shape[-1] not in HEAD_DIMS:
        return False
    if not (q.stride(-1) == k.stride(-1) == v.stride(-1) == 1):
        return False
    esz = q.element_size()
    for t in (q, k, v):
        if any((s * esz) % 16 != 0 for s in t.stride()[:3]):
            return False
    return True


def _common_ok(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dtype: torch.dtype) -> bool:
    return _layout_ok(q, k, v, dtype) and all(t.data_ptr() % 16 == 0 for t in (q, k, v))


def is_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool) -> bool:
    """Whether the FP32-I/O causal kernel supports this exact invocation."""
    return bool(causal) and _common_ok(q, k, v, torch.float32)


def is_fp16_supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool) -> bool:
    """Whether the FP16-I/O causal kernel supports this exact invocation."""
    return bool(causal) and _common_ok(q, k, v, torch.float16)


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    *,
    causal: bool = True,
    key_valid: Optional[torch.Tensor] = None,
    out_dtype: Optional[torch.dtype] = None,
    variant: int = 0,
) -> torch.Tensor:
    """Flash attention ``softmax(q k^T * scale [+ masks]) v`` -> contiguous ``[B, S, H, hd]``.

    ``key_valid`` is an optional bool ``[B, S]`` key-padding mask (True = may be
    attended).  ``out_dtype`` defaults to the input dtype.
    """
    if not _layout_ok(q, k, v, q.dtype) or q.dtype not in (torch.float16, torch.float32):
        raise ValueError(f"unsupported custom-attention input: shape={tuple(q.shape)}, dtype={q.dtype}")
    batch, heads, seq_len, head_dim = q.shape
    out_dtype = q.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.float16, torch.float32):
        raise ValueError(f"unsupported attention output dtype {out_dtype}")
    mask_u8 = None
    if key_valid is not None:
        if key_valid.shape != (batch, seq_len) or key_valid.device != q.device:
            raise ValueError("key_valid must be a [batch, seq_len] mask on the input device")
        mask_u8 = key_valid.to(torch.uint8).contiguous()
    return _ops.attention(q, k, v, mask_u8, float(scale), bool(causal), F16 if out_dtype == torch.float16 else F32,
                          int(variant))


def attention_prescaled(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    causal: bool = True,
    key_valid: Optional[torch.Tensor] = None,
    variant: int = 0,
) -> torch.Tensor:
    """``attention`` for FP16 inputs whose q already holds ``q * scale * log2(e)`` (rounded to
    FP16 once, by ``hip_linear.mixed_linear_q_scaled``): the 32x32 kernel (head dims 32 and
    64; ``variant`` 0 or 6-8) without the per-score scale.  Output FP16 ``[B, S, H, hd]``."""
    if not _layout_ok(q, k, v, q.dtype) or q.dtype != torch.float16 or q.shape[-1] not in (32, 64):
        raise ValueError(f"unsupported pre-scaled attention input: shape={tuple(q.shape)}, dtype={q.dtype}")
    if int(variant) not in (0, 6, 7, 8):
        raise ValueError(f"pre-scaled attention runs variants 6-8 (got {variant})")
    batch, heads, seq_len, head_dim = q.shape
    mask_u8 = None
    if key_valid is not None:
        if key_valid.shape != (batch, seq_len) or key_valid.device != q.device:
            raise ValueError("key_valid must be a [batch, seq_len] mask on the input device")
        mask_u8 = key_valid.to(torch.uint8).contiguous()
    return _ops.attention_prescaled(q, k, v, mask_u8, bool(causal), F16, int(variant))


def launch_causal_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: float,
    *,
    block_m: int = 64,
    block_n: int = 32,
    num_warps: int = 4,
    num_stages: int = 2,
    dot_precision: str = "tf32",
    variant: int = 0,
) -> torch.Tensor:
    """Explicit-configuration entry kept for call-site compatibility (FP32 I/O, causal)."""
    if not is_supported(q, k, v, causal=True):
        raise ValueError(f"unsupported custom-attention input: shape={tuple(q.shape)}, dtype={q.dtype}")
    return attention(q, k, v, scale, causal=True, variant=variant)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal attention for FP32 q/k/v, FP32 ``[B, S, H, hd]`` output."""
    return launch_causal_attention(q, k, v, scale)


def fp16_causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Causal attention for FP16 q/k/v, FP16 ``[B, S, H, hd]`` output."""
    if not is_fp16_supported(q, k, v, causal=True):
        raise ValueError(f"unsupported FP16 custom-attention input: {tuple(q.shape)}")
    return attention(q, k, v, scale, causal=True)


def default_scale(head_dim: int) -> float:
    return head_dim ** -0.5 if head_dim > 0 else math.nan
