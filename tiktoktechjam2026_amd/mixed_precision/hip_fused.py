"""Cross-operator fusions of the HIP forward (no single reference function corresponds).

``fused_attention_layer_tail`` runs the causal (or full) attention of head dim 32 (or 16 at
d_model 32 and 64) in the same kernel, from the packed QKV projection, for sequences whose
length is a multiple of its 64-row tiles (no key mask): one launch per layer instead of two.

``fused_layer_tail`` composes, with the same rounding points, the reference's
``mixed_linear_add_layer_norm`` (attention output projection + residual + LN2),
``mixed_ffn_add_layer_norm`` (FFN + residual + next LN) and the next layer's
``mixed_linear`` QKV projection (``mixed_precision/transformer.py:196-222,
540-560, 88-120``), keeping every intermediate on chip.  ``layer_norm_qkv``
fuses the initial ``norm1`` + cast (``:484-486``) with the first QKV projection.
Both validate shapes, dtypes and layouts in Python (``ValueError``) and call
one ``torch.library`` custom operator (``tiktoktechjam2026_amd/_ops.py``) that
launches on torch's current stream.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from .. import _ops
from ..dispatch import ATTENTION_TAIL_ROWS, LAYER_TAIL_SHAPES, LAYERNORM_QKV_WIDTHS, attention_tail_supported
from .hip_linear import _fp16_linear_ok, _gpu, _norm_ok


def layer_tail_supported(d_model: int, ffn_dim: int) -> bool:
    """(d_model, ffn_dim) pairs the layer-tail kernel is built for (``mpk_layer_tail_supported``)."""
    return (int(d_model), int(ffn_dim)) in LAYER_TAIL_SHAPES


def layer_norm_qkv_supported(d_model: int) -> bool:
    """d_model values of the LayerNorm + QKV kernel (``mpk_layernorm_qkv_supported``)."""
    return int(d_model) in LAYERNORM_QKV_WIDTHS


def layer_norm_qkv(
    x: torch.Tensor, norm: nn.LayerNorm, qkv_proj: nn.Linear, *, variant: int = 0, q_scale: Optional[float] = None
) -> torch.Tensor:
    """``fp16(LayerNorm(x)) @ Wqkv^T + b`` -> FP16 ``[..., 3D]`` (FP32 statistics and accumulation).

    ``q_scale``: the q columns leave multiplied by it (in FP32, before the FP16 rounding), the
    input ``attention_prescaled`` takes with ``q_scale = scale * log2(e)``."""
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
    return _ops.layer_norm_qkv(x, norm.weight, norm.bias, qkv_proj.weight, qkv_proj.bias, float(norm.eps),
                               int(variant), _q_scale(q_scale))


def _q_scale(q_scale: Optional[float]) -> float:
    """The custom ops' encoding: 0.0 for no q scaling, else a finite nonzero FP32 factor."""
    if q_scale is None:
        return 0.0
    q = float(q_scale)
    if not math.isfinite(q) or q == 0.0:
        raise ValueError("q_scale must be finite and nonzero")
    return q


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
    q_scale: Optional[float] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention output projection through the next layer's QKV projection in one kernel.

    Returns ``(residual_out, qkv)`` with ``qkv`` FP16 ``[..., 3D]``, or, when
    ``next_qkv_proj`` is None (last layer), ``(residual_out, normalized)`` with
    ``normalized = next_norm(residual_out)`` in FP32.  ``q_scale`` as for ``layer_norm_qkv``
    (ignored for the last layer, which has no next QKV).
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
    tensors = [out_proj.weight, out_proj.bias, norm2.weight, norm2.bias, ffn_in.weight, ffn_in.bias,
               ffn_out.weight, ffn_out.bias, next_norm.weight, next_norm.bias]
    return _ops.layer_tail(
        ctx, residual, tensors, None if last else next_qkv_proj.weight, None if last else next_qkv_proj.bias,
        float(norm2.eps), float(next_norm.eps), int(variant), 0.0 if last else _q_scale(q_scale),
    )


def attention_layer_tail_supported(d_model: int, ffn_dim: int, heads: int, seq_len: int) -> bool:
    """Shapes of ``mpk_attention_layer_tail`` (``mpk_attention_layer_tail_supported`` and
    ``_rows``; the tables are checked against the library by the tests): head dim 32 on a
    layer-tail shape or 16 at d_model 32 / 64, whole 64-row tiles."""
    s = int(seq_len)
    return attention_tail_supported(d_model, ffn_dim, heads) and s > 0 and s % ATTENTION_TAIL_ROWS == 0


def fused_attention_layer_tail(
    qkv: torch.Tensor,
    residual: torch.Tensor,
    heads: int,
    scale: float,
    causal: bool,
    out_proj: nn.Linear,
    norm2: nn.LayerNorm,
    ffn_in: nn.Linear,
    ffn_out: nn.Linear,
    next_norm: nn.LayerNorm,
    next_qkv_proj: Optional[nn.Linear] = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention over this layer's packed ``qkv [B, S, 3D]`` (FP16) and everything after it up to
    the next layer's QKV projection, in one kernel.

    Same arithmetic as ``attention`` (variant 1: 16x16 kernel, 64-key tiles) followed by
    ``fused_layer_tail``.  Returns ``(residual_out, next qkv)``, or ``(residual_out,
    next_norm(residual_out))`` in FP32 when ``next_qkv_proj`` is None (last layer).
    """
    ok = _gpu(qkv) and qkv.dtype == torch.float16 and qkv.dim() == 3 and qkv.is_contiguous()
    d = residual.shape[-1] if residual.dim() else 0
    f = ffn_in.out_features
    last = next_qkv_proj is None
    if not (
        ok
        and _gpu(residual)
        and residual.dtype == torch.float32
        and residual.dim() == 3
        and residual.is_contiguous()
        and qkv.shape == (*residual.shape[:-1], 3 * d)
        and out_proj.in_features == out_proj.out_features == d
        and ffn_in.in_features == d
        and ffn_out.in_features == f
        and ffn_out.out_features == d
        and all(_fp16_linear_ok(m) for m in (out_proj, ffn_in, ffn_out))
        and _norm_ok(norm2, d)
        and _norm_ok(next_norm, d)
        and (last or (_fp16_linear_ok(next_qkv_proj) and next_qkv_proj.in_features == d
                      and next_qkv_proj.out_features == 3 * d))
        and attention_layer_tail_supported(d, f, heads, residual.shape[1])
    ):
        raise ValueError("unsupported fused attention layer-tail inputs")
    tensors = [out_proj.weight, out_proj.bias, norm2.weight, norm2.bias, ffn_in.weight, ffn_in.bias,
               ffn_out.weight, ffn_out.bias, next_norm.weight, next_norm.bias]
    return _ops.attention_layer_tail(
        qkv, residual, tensors, None if last else next_qkv_proj.weight, None if last else next_qkv_proj.bias,
        int(heads), float(scale), bool(causal), float(norm2.eps), float(next_norm.eps),
    )
