"""Projection / fusion operators backed by the gfx950 HIP kernels in ``libmpk.so``.

Same names, positional/keyword signatures and error behaviour as the
reference's ``mixed_precision/triton_linear.py`` (``mixed_linear`` :221,
``mixed_linear_add_layer_norm`` :272, ``mixed_ffn_add_layer_norm`` :327,
``mixed_add_layer_norm`` :381) and ``fused_add_layer_norm``
(``torch_transformer_benchmark.py:72``).  The Triton tuning keywords
(``block_m``, ``block_n``, ``block_k``, ``group_m``, ``num_warps``,
``num_stages``) are accepted for call-site compatibility and ignored: tile
shapes come from the HIP dispatch table, or from the extra ``variant`` keyword.

Every wrapper validates shapes, dtypes and layouts in Python and raises
``ValueError`` before launching, then calls one ``torch.library`` custom
operator (``tiktoktechjam2026_amd/_ops.py``), which checks alignment,
allocates the outputs with ``torch.empty`` on the input device and launches on
torch's current HIP stream.  The validation reads only shapes, dtypes and
strides, so ``torch.compile`` traces the wrappers into one graph of custom
operators.  There is no CPU or PyTorch fallback: non-GPU tensors are rejected.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .. import _ops
from .._lib import F16, F32


def _code(dtype: torch.dtype) -> int:
    return F16 if dtype == torch.float16 else F32


def _gpu(t: torch.Tensor) -> bool:
    return t.is_cuda and t.is_contiguous()


def _fp16_linear_ok(linear: nn.Linear) -> bool:
    return (
        linear.weight.is_cuda
        and linear.weight.dtype == torch.float16
        and linear.weight.is_contiguous()
        and linear.bias is not None
        and linear.bias.dtype == torch.float16
        and linear.bias.is_contiguous()
    )


def _norm_ok(norm: nn.LayerNorm, width: int) -> bool:
    return (
        tuple(norm.normalized_shape) == (width,)
        and norm.weight is not None
        and norm.bias is not None
        and norm.weight.is_cuda
        and norm.weight.dtype == torch.float32
        and norm.bias.dtype == torch.float32
        and norm.weight.is_contiguous()
        and norm.bias.is_contiguous()
    )


def mixed_linear(
    x: torch.Tensor,
    linear: nn.Linear,
    *,
    output_dtype: torch.dtype,
    fuse_gelu: bool = False,
    block_m: int = 64,
    block_n: int = 64,
    block_k: int = 32,
    group_m: int = 8,
    num_warps: int = 4,
    num_stages: int = 3,
    variant: int = 0,
) -> torch.Tensor:
    """``act(fp16(x) @ W^T + b)`` with FP32 accumulation; act = exact GELU if ``fuse_gelu``."""
    if not (
        _gpu(x)
        and x.dtype in (torch.float16, torch.float32)
        and _fp16_linear_ok(linear)
        and output_dtype in (torch.float16, torch.float32)
        and x.shape[-1] == linear.in_features
        and linear.in_features % 8 == 0
        and linear.out_features % 8 == 0
    ):
        raise ValueError("unsupported mixed projection inputs")
    return _ops.linear(x, linear.weight, linear.bias, _code(output_dtype), bool(fuse_gelu), int(variant))


def mixed_linear_q_scaled(
    x: torch.Tensor, linear: nn.Linear, q_cols: int, q_scale: float, *, variant: int = 0
) -> torch.Tensor:
    """``fp16(x) @ W^T + b`` -> FP16, with output columns below ``q_cols`` multiplied by
    ``q_scale`` in FP32 before the FP16 rounding: the packed QKV projection with the attention's
    ``scale * log2(e)`` folded into q, for ``attention_prescaled`` (no reference counterpart:
    the reference scales the scores, ``custom_kernel/triton_attention.py:85``)."""
    if not (
        _gpu(x)
        and x.dtype in (torch.float16, torch.float32)
        and _fp16_linear_ok(linear)
        and x.shape[-1] == linear.in_features
        and linear.in_features % 8 == 0
        and linear.out_features % 8 == 0
        and 0 <= int(q_cols) <= linear.out_features
        and int(q_cols) % 8 == 0
    ):
        raise ValueError("unsupported mixed projection inputs")
    return _ops.linear_qscaled(x, linear.weight, linear.bias, _code(torch.float16), int(q_cols), float(q_scale),
                               int(variant))


def mixed_linear_residual(
    x: torch.Tensor,
    linear: nn.Linear,
    residual: torch.Tensor,
    *,
    out: Optional[torch.Tensor] = None,
    variant: int = 0,
) -> torch.Tensor:
    """``fp16(x) @ W^T + b + residual`` in FP32 (the projection and residual add of the unfused route).

    ``out`` may be ``residual`` itself for an in-place add.
    """
    if not (
        _gpu(x)
        and x.dtype in (torch.float16, torch.float32)
        and _fp16_linear_ok(linear)
        and x.shape[-1] == linear.in_features
        and linear.in_features % 8 == 0
        and linear.out_features % 8 == 0
        and _gpu(residual)
        and residual.dtype == torch.float32
        and residual.is_contiguous()
        and residual.shape == (*x.shape[:-1], linear.out_features)
        and (out is None or (_gpu(out) and out.dtype == torch.float32 and out.is_contiguous()
                             and out.shape == residual.shape))
    ):
        raise ValueError("unsupported mixed projection/residual inputs")
    if out is None:
        return _ops.linear_residual(x, linear.weight, linear.bias, residual, int(variant))
    _ops.linear_residual_into(x, linear.weight, linear.bias, residual, out, int(variant))
    return out


LN_FUSED_WIDTHS = (32, 64, 128, 256, 512)


def mixed_linear_add_layer_norm(
    x: torch.Tensor,
    linear: nn.Linear,
    residual: torch.Tensor,
    norm: nn.LayerNorm,
    *,
    block_m: int = 64,
    block_k: int = 32,
    num_warps: int = 4,
    num_stages: int = 2,
    normalized_dtype: torch.dtype = torch.float32,
    variant: int = 0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``R' = fp16(x) @ W^T + b + residual``; ``N' = LayerNorm(R')``; returns ``(R', N')``."""
    if not (
        _gpu(x)
        and x.dtype in (torch.float16, torch.float32)
        and _gpu(residual)
        and residual.dtype == torch.float32
        and x.shape[:-1] == residual.shape[:-1]
        and x.shape[-1] == residual.shape[-1]
        and x.shape[-1] in LN_FUSED_WIDTHS
        and linear.in_features == linear.out_features == x.shape[-1]
        and _fp16_linear_ok(linear)
        and _norm_ok(norm, x.shape[-1])
        and normalized_dtype in (torch.float16, torch.float32)
    ):
        raise ValueError("unsupported fused projection/residual/LayerNorm inputs")
    return _ops.linear_residual_layer_norm(
        x, linear.weight, linear.bias, residual, norm.weight, norm.bias, float(norm.eps), _code(normalized_dtype),
        int(variant),
    )


WIDE_LN_EPILOGUE_WIDTHS = (256, 512)


def mixed_linear_residual_layer_norm(
    x: torch.Tensor,
    linear: nn.Linear,
    residual: torch.Tensor,
    norm: nn.LayerNorm,
    *,
    normalized_dtype: torch.dtype = torch.float32,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``R' = fp16(x) @ W^T + b + residual``; ``N' = LayerNorm(R')`` for any input width.

    The wide-route counterpart of ``mixed_linear_add_layer_norm`` (whose
    projection is square): the out-projection or the FFN-output projection,
    its residual add and the next LayerNorm (reference generic route,
    ``mixed_precision/transformer.py:664-690``) run as one kernel on GEMM tiles
    that hold whole rows.  ``linear.out_features`` must be 256 or 512.  Returns
    ``(R', N')``.
    """
    n_features = linear.out_features
    if not (
        _gpu(x)
        and x.dtype in (torch.float16, torch.float32)
        and _gpu(residual)
        and residual.dtype == torch.float32
        and x.shape[:-1] == residual.shape[:-1]
        and x.shape[-1] == linear.in_features
        and linear.in_features % 8 == 0
        and residual.shape[-1] == n_features
        and n_features in WIDE_LN_EPILOGUE_WIDTHS
        and _fp16_linear_ok(linear)
        and _norm_ok(norm, n_features)
        and normalized_dtype in (torch.float16, torch.float32)
    ):
        raise ValueError("unsupported projection/residual/LayerNorm inputs")
    return _ops.linear_add_layer_norm(
        x, linear.weight, linear.bias, residual, norm.weight, norm.bias, float(norm.eps), _code(normalized_dtype)
    )


def mixed_ffn_add_layer_norm(
    x: torch.Tensor,
    linear_in: nn.Linear,
    linear_out: nn.Linear,
    residual: torch.Tensor,
    norm: nn.LayerNorm,
    *,
    block_m: int = 16,
    num_warps: int = 4,
    num_stages: int = 2,
    normalized_dtype: torch.dtype = torch.float32,
    variant: int = 0,
    out: Optional[torch.Tensor] = None,
    store_residual: bool = True,
) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
    """Whole FFN (exact GELU on the FP32 accumulator) + residual + LayerNorm; returns ``(R', N')``.
    ``out``: optional contiguous tensor of ``residual``'s shape and ``normalized_dtype`` that
    receives N' (then returned as N'); ``store_residual=False`` skips R' (returned as None)."""
    d = x.shape[-1] if x.dim() > 0 else 0
    if not (
        _gpu(x)
        and x.dtype in (torch.float16, torch.float32)
        and _gpu(residual)
        and residual.dtype == torch.float32
        and x.shape == residual.shape
        and d in LN_FUSED_WIDTHS
        and linear_in.in_features == d
        and linear_out.out_features == d
        and linear_in.out_features == linear_out.in_features
        and linear_in.out_features % 32 == 0
        and _fp16_linear_ok(linear_in)
        and _fp16_linear_ok(linear_out)
        and _norm_ok(norm, d)
        and normalized_dtype in (torch.float16, torch.float32)
        and (
            out is None
            or (_gpu(out) and out.dtype == normalized_dtype and out.shape == residual.shape and out.is_contiguous())
        )

    ):
        raise ValueError("unsupported fused FFN inputs")
    if out is not None:
        residual_out = _ops.ffn_residual_layer_norm_into(
            x, linear_in.weight, linear_in.bias, linear_out.weight, linear_out.bias, residual, norm.weight,
            norm.bias, float(norm.eps), int(variant), out, bool(store_residual),
        )
        return (residual_out if store_residual else None), out
    if not store_residual:
        return None, _ops.ffn_residual_layer_norm_final(
            x, linear_in.weight, linear_in.bias, linear_out.weight, linear_out.bias, residual, norm.weight,
            norm.bias, float(norm.eps), _code(normalized_dtype), int(variant),
        )
    return _ops.ffn_residual_layer_norm(
        x, linear_in.weight, linear_in.bias, linear_out.weight, linear_out.bias, residual, norm.weight, norm.bias,
        float(norm.eps), _code(normalized_dtype), int(variant),
    )


def _add_layer_norm(
    x: torch.Tensor,
    update: Optional[torch.Tensor],
    norm: nn.LayerNorm,
    normalized_dtype: torch.dtype,
    message: str,
) -> Tuple[Optional[torch.Tensor], torch.Tensor]:
    width = x.shape[-1] if x.dim() > 0 else 0
    if not (
        _gpu(x)
        and x.dtype == torch.float32
        and (update is None or (_gpu(update) and update.dtype == torch.float32 and update.shape == x.shape))
        and normalized_dtype in (torch.float16, torch.float32)
        and width > 0
        and width % 4 == 0
        and width <= 2048
        and _norm_ok(norm, width)
    ):
        raise ValueError(message)
    if update is None:
        return None, _ops.layer_norm(x, norm.weight, norm.bias, float(norm.eps), _code(normalized_dtype))
    return _ops.add_layer_norm(x, update, norm.weight, norm.bias, float(norm.eps), _code(normalized_dtype))


def mixed_add_layer_norm(
    x: torch.Tensor,
    update: torch.Tensor,
    norm: nn.LayerNorm,
    *,
    normalized_dtype: torch.dtype,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """FP32 ``residual = x + update`` and its LayerNorm in FP16 or FP32; returns ``(residual, normalized)``."""
    residual, normalized = _add_layer_norm(x, update, norm, normalized_dtype, "unsupported mixed LayerNorm inputs")
    assert residual is not None
    return residual, normalized


def fused_add_layer_norm(
    x: torch.Tensor, update: torch.Tensor, norm: nn.LayerNorm
) -> Tuple[torch.Tensor, torch.Tensor]:
    """FP32 residual add + LayerNorm with an FP32 normalized output (reference K5 contract)."""
    residual, normalized = _add_layer_norm(
        x, update, norm, torch.float32, "unsupported fused residual/LayerNorm inputs"
    )
    assert residual is not None
    return residual, normalized


def layer_norm(x: torch.Tensor, norm: nn.LayerNorm, *, normalized_dtype: torch.dtype) -> torch.Tensor:
    """Plain LayerNorm of an FP32 stream with an FP16 or FP32 output (the initial ``norm1`` + cast)."""
    _, normalized = _add_layer_norm(x, None, norm, normalized_dtype, "unsupported LayerNorm inputs")
    return normalized
