"""Projection / fusion operators backed by the gfx950 HIP kernels in ``libmpk.so``.

Same names, positional/keyword signatures and error behaviour as the
reference's ``mixed_precision/triton_linear.py`` (``mixed_linear`` :221,
``mixed_linear_add_layer_norm`` :272, ``mixed_ffn_add_layer_norm`` :327,
``mixed_add_layer_norm`` :381) and ``fused_add_layer_norm``
(``torch_transformer_benchmark.py:72``).  The Triton tuning keywords
(``block_m``, ``block_n``, ``block_k``, ``group_m``, ``num_warps``,
``num_stages``) are accepted for call-site compatibility and ignored: tile
shapes come from the HIP dispatch table, or from the extra ``variant`` keyword.

Every wrapper validates its inputs in Python and raises ``ValueError`` before
launching, allocates its outputs with ``torch.empty`` on the input device,
and launches on torch's current HIP stream.  There is no CPU or PyTorch
fallback: non-GPU tensors are rejected.
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
import torch.nn as nn

from .. import _lib


def _aligned(*tensors: torch.Tensor) -> bool:
    return all(t.data_ptr() % 16 == 0 for t in tensors)


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
    in_features = linear.in_features
    out_features = linear.out_features
    n_rows = x.numel() // in_features
    output = torch.empty((*x.shape[:-1], out_features), device=x.device, dtype=output_dtype)
    if not _aligned(x, linear.weight, linear.bias, output):
        raise ValueError("unsupported mixed projection inputs (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_linear(
            x.data_ptr(), _lib.dtype_code(x.dtype), linear.weight.data_ptr(), linear.bias.data_ptr(),
            output.data_ptr(), _lib.dtype_code(output_dtype), 1 if fuse_gelu else 0, n_rows, out_features,
            in_features, int(variant), _lib.stream_handle(x.device),
        ),
        "mpk_linear",
    )
    return output


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
    n_rows = x.numel() // linear.in_features
    output = torch.empty_like(residual) if out is None else out
    if not _aligned(x, linear.weight, linear.bias, residual, output):
        raise ValueError("unsupported mixed projection/residual inputs (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_linear_residual(
            x.data_ptr(), _lib.dtype_code(x.dtype), linear.weight.data_ptr(), linear.bias.data_ptr(),
            residual.data_ptr(), output.data_ptr(), n_rows, linear.out_features, linear.in_features, int(variant),
            _lib.stream_handle(x.device),
        ),
        "mpk_linear_residual",
    )
    return output


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
    n_features = x.shape[-1]
    n_rows = x.numel() // n_features
    residual_out = torch.empty_like(residual)
    normalized_out = torch.empty_like(residual, dtype=normalized_dtype)
    if not _aligned(x, residual, linear.weight, linear.bias, norm.weight, norm.bias, residual_out, normalized_out):
        raise ValueError("unsupported fused projection/residual/LayerNorm inputs (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_linear_residual_layernorm(
            x.data_ptr(), _lib.dtype_code(x.dtype), linear.weight.data_ptr(), linear.bias.data_ptr(),
            residual.data_ptr(), norm.weight.data_ptr(), norm.bias.data_ptr(), residual_out.data_ptr(),
            normalized_out.data_ptr(), _lib.dtype_code(normalized_dtype), n_rows, n_features, float(norm.eps),
            int(variant), _lib.stream_handle(x.device),
        ),
        "mpk_linear_residual_layernorm",
    )
    return residual_out, normalized_out


WIDE_LN_EPILOGUE_WIDTH = 256


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
    ``mixed_precision/transformer.py:664-690``) run as one kernel on 256 x 256
    GEMM tiles.  ``linear.out_features`` must be 256.  Returns ``(R', N')``.
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
        and residual.shape[-1] == n_features == WIDE_LN_EPILOGUE_WIDTH
        and _fp16_linear_ok(linear)
        and _norm_ok(norm, n_features)
        and normalized_dtype in (torch.float16, torch.float32)
    ):
        raise ValueError("unsupported projection/residual/LayerNorm inputs")
    n_rows = residual.numel() // n_features
    residual_out = torch.empty_like(residual)
    normalized_out = torch.empty_like(residual, dtype=normalized_dtype)
    if not _aligned(x, residual, linear.weight, linear.bias, norm.weight, norm.bias, residual_out, normalized_out):
        raise ValueError("unsupported projection/residual/LayerNorm inputs (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_linear_add_layernorm(
            x.data_ptr(), _lib.dtype_code(x.dtype), linear.weight.data_ptr(), linear.bias.data_ptr(),
            residual.data_ptr(), norm.weight.data_ptr(), norm.bias.data_ptr(), residual_out.data_ptr(),
            normalized_out.data_ptr(), _lib.dtype_code(normalized_dtype), n_rows, n_features,
            linear.in_features, float(norm.eps), _lib.stream_handle(x.device),
        ),
        "mpk_linear_add_layernorm",
    )
    return residual_out, normalized_out


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
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Whole FFN (exact GELU on the FP32 accumulator) + residual + LayerNorm; returns ``(R', N')``."""
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
    ):
        raise ValueError("unsupported fused FFN inputs")
    ffn_dim = linear_in.out_features
    n_rows = x.numel() // d
    residual_out = torch.empty_like(residual)
    normalized_out = torch.empty_like(residual, dtype=normalized_dtype)
    if not _aligned(
        x, residual, linear_in.weight, linear_in.bias, linear_out.weight, linear_out.bias, norm.weight, norm.bias,
        residual_out, normalized_out,
    ):
        raise ValueError("unsupported fused FFN inputs (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_ffn_residual_layernorm(
            x.data_ptr(), _lib.dtype_code(x.dtype), linear_in.weight.data_ptr(), linear_in.bias.data_ptr(),
            linear_out.weight.data_ptr(), linear_out.bias.data_ptr(), residual.data_ptr(), norm.weight.data_ptr(),
            norm.bias.data_ptr(), residual_out.data_ptr(), normalized_out.data_ptr(),
            _lib.dtype_code(normalized_dtype), n_rows, d, ffn_dim, float(norm.eps), int(variant),
            _lib.stream_handle(x.device),
        ),
        "mpk_ffn_residual_layernorm",
    )
    return residual_out, normalized_out


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
    n_rows = x.numel() // width
    residual = torch.empty_like(x) if update is not None else None
    normalized = torch.empty_like(x, dtype=normalized_dtype)
    tensors = [x, norm.weight, norm.bias, normalized] + ([update, residual] if update is not None else [])
    if not _aligned(*tensors):
        raise ValueError(message + " (16-byte alignment)")
    lib = _lib.load()
    _lib.check(
        lib.mpk_layernorm(
            x.data_ptr(), None if update is None else update.data_ptr(), norm.weight.data_ptr(), norm.bias.data_ptr(),
            None if residual is None else residual.data_ptr(), normalized.data_ptr(),
            _lib.dtype_code(normalized_dtype), n_rows, width, float(norm.eps), _lib.stream_handle(x.device),
        ),
        "mpk_layernorm",
    )
    return residual, normalized


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
