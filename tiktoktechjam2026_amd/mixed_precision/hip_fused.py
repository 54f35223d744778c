"""Cross-operator fusions of the HIP forward (no single reference function corresponds).

``fused_layer_tail`` composes, with the same rounding points, the reference's
``mixed_linear_add_layer_norm`` (attention output projection + residual + LN2),
``mixed_ffn_add_layer_norm`` (FFN + residual + next LN) and the next layer's
``mixed_linear`` QKV projection (``mixed_precision/transformer.py:196-222,
540-560, 88-120``), keeping every intermediate on chip.  ``layer_norm_qkv``
fuses the initial ``norm1`` + cast (``:484-486``) with the first QKV projection.
Both validate in Python (``ValueError``) and launch on torch's current stream.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .. import _lib
from .hip_linear import _aligned, _fp16_linear_ok, _gpu, _norm_ok


def layer_tail_supported(d_model: int, ffn_dim: int) -> bool:
    return bool(_lib.load().mpk_layer_tail_supported(int(d_model), int(ffn_dim)))


def layer_norm_qkv_supported(d_model: int) -> bool:
    return bool(_lib.load().mpk_layernorm_qkv_supported(int(d_model)))


def layer_norm_qkv(x: torch.Tensor, norm: nn.LayerNorm, qkv_proj: nn.Linear, *, variant: int = 0) -> torch.Tensor:
    """``fp16(LayerNorm(x)) @ Wqkv^T + b`` -> FP16 ``[..., 3D]`` (FP32 statistics and accumulation)."""
    d = x.shape[-1] if x.dim() else 0
    if not (
        _gpu(x)
        and x.dtype == torch.float32
        and _norm_ok(norm, d)
        and _fp16_linear_ok(qkv_proj)
        and qkv_proj.in_features == d
        and qkv_proj.out_features == 3 * d
        and layer_norm_qkv_supported(d)
    ):
        raise ValueError("unsupported LayerNorm/QKV inputs")
    rows = x.numel() // d
    out = torch.empty((*x.shape[:-1], 3 * d), device=x.device, dtype=torch.float16)
    if not _aligned(x, norm.weight, norm.bias, qkv_proj.weight, qkv_proj.bias, out):
        raise ValueError("unsupported LayerNorm/QKV inputs (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_layernorm_qkv(
            x.data_ptr(), norm.weight.data_ptr(), norm.bias.data_ptr(), qkv_proj.weight.data_ptr(),
            qkv_proj.bias.data_ptr(), out.data_ptr(), rows, d, float(norm.eps), int(variant),
            _lib.stream_handle(x.device),
        ),
        "mpk_layernorm_qkv",
    )
    return out


def fused_layer_tail(
    ctx: torch.Tensor,
    residual: torch.Tensor,
    out_proj: nn.Linear,
    norm2: nn.LayerNorm,
    ffn_in: nn.Linear,
    ffn_out: nn.Linear,
    next_norm: nn.LayerNorm,
    next_qkv_proj: Optional[nn.Linear] = None,
    *,
    variant: int = 0,
    out: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention output projection through the next layer's QKV projection in one kernel.

    Returns ``(residual_out, qkv)`` with ``qkv`` FP16 ``[..., 3D]``, or, when
    ``next_qkv_proj`` is None (last layer), ``(residual_out, normalized)`` with
    ``normalized = next_norm(residual_out)`` in FP32.  ``out`` optionally
    supplies the second result's storage (e.g. a slice of a preallocated output).
    """
    d = ctx.shape[-1] if ctx.dim() else 0
    f = ffn_in.out_features
    last = next_qkv_proj is None
    if not (
        _gpu(ctx)
        and ctx.dtype == torch.float16
        and _gpu(residual)
        and residual.dtype == torch.float32
        and residual.shape == ctx.shape
        and out_proj.in_features == out_proj.out_features == d
        and ffn_in.in_features == d
        and ffn_out.in_features == f
        and ffn_out.out_features == d
        and all(_fp16_linear_ok(m) for m in (out_proj, ffn_in, ffn_out))
        and _norm_ok(norm2, d)
        and _norm_ok(next_norm, d)
        and (last or (_fp16_linear_ok(next_qkv_proj) and next_qkv_proj.in_features == d
                      and next_qkv_proj.out_features == 3 * d))
        and layer_tail_supported(d, f)
    ):
        raise ValueError("unsupported fused layer-tail inputs")
    rows = ctx.numel() // d
    residual_out = torch.empty_like(residual)
    shape = ctx.shape if last else (*ctx.shape[:-1], 3 * d)
    dtype = torch.float32 if last else torch.float16
    if out is None:
        out = torch.empty(shape, device=ctx.device, dtype=dtype)
    elif tuple(out.shape) != tuple(shape) or out.dtype != dtype or not _gpu(out):
        raise ValueError("fused layer-tail `out` has the wrong shape, dtype or layout")
    tensors = [ctx, residual, out_proj.weight, out_proj.bias, norm2.weight, norm2.bias, ffn_in.weight, ffn_in.bias,
               ffn_out.weight, ffn_out.bias, next_norm.weight, next_norm.bias, residual_out, out]
    if not last:
        tensors += [next_qkv_proj.weight, next_qkv_proj.bias]
    if not _aligned(*tensors):
        raise ValueError("unsupported fused layer-tail inputs (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_layer_tail(
            ctx.data_ptr(), residual.data_ptr(), out_proj.weight.data_ptr(), out_proj.bias.data_ptr(),
            norm2.weight.data_ptr(), norm2.bias.data_ptr(), ffn_in.weight.data_ptr(), ffn_in.bias.data_ptr(),
            ffn_out.weight.data_ptr(), ffn_out.bias.data_ptr(), next_norm.weight.data_ptr(),
            next_norm.bias.data_ptr(), None if last else next_qkv_proj.weight.data_ptr(),
            None if last else next_qkv_proj.bias.data_ptr(), residual_out.data_ptr(), out.data_ptr(),
            1 if last else 0, rows, d, f, float(norm2.eps), float(next_norm.eps), int(variant),
            _lib.stream_handle(ctx.device),
        ),
        "mpk_layer_tail",
    )
    return residual_out, out
