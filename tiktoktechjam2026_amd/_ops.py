"""``torch.library`` custom operators over the C ABI (``include/mpk.h``).

Each operator is opaque to ``torch.compile``: Dynamo records it as one node,
Inductor calls it as an external kernel, and the fake (meta) implementation
gives the output shapes and dtypes without touching the device.  That is what
lets the reference CLI's default ``torch.compile(model, mode="reduce-overhead")``
(``mixed_precision_benchmark.py:86-90`` -> ``torch_transformer_benchmark.py:800-805``)
trace the module's forward in one graph and capture it in a HIP graph.

The real implementations check 16-byte alignment (``ValueError``, as the
Python wrappers did before launching), allocate the outputs with
``torch.empty`` on the input's device and launch on torch's current stream.
Shape, dtype and layout validation stays in the public wrappers
(``mixed_precision/hip_linear.py``, ``hip_fused.py``,
``custom_kernel/hip_attention.py``), which raise the reference's
``ValueError`` messages before any operator is called.

dtype arguments are the C ABI codes: 0 = FP32, 1 = FP16.
"""


from typing import List, Optional, Tuple

import torch

from . import _lib

_DTYPES = {_lib.F32: torch.float32, _lib.F16: torch.float16}


def _dtype(code: int) -> torch.dtype:
    try:
        return _DTYPES[int(code)]
    except KeyError:
        raise ValueError(f"unknown dtype code {code}") from None


def _require_aligned(message: str, *tensors: Optional[torch.Tensor]) -> None:
    if any(t is not None and t.data_ptr() % 16 != 0 for t in tensors):
        raise ValueError(message + " (16-byte alignment)")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _rows(t: torch.Tensor, width: int) -> int:
    return t.numel() // width if width else 0


# --------------------------------------------------------------------------- LayerNorm


@torch.library.custom_op("mpk::layer_norm", mutates_args=())
def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float, out_dtype: int) -> torch.Tensor:
    """``LayerNorm(x)`` of an FP32 stream with FP32 statistics (``mpk_layernorm``, no update)."""
    d = x.shape[-1]
    out = torch.empty(x.shape, device=x.device, dtype=_dtype(out_dtype))
    _require_aligned("unsupported LayerNorm inputs", x, weight, bias, out)
    _lib.check(
        _lib.load().mpk_layernorm(
            x.data_ptr(), None, weight.data_ptr(), bias.data_ptr(), None, out.data_ptr(), int(out_dtype),
            _rows(x, d), d, float(eps), _lib.stream_handle(x.device),
        ),
        "mpk_layernorm",
    )
    return out


@layer_norm.register_fake
def _(x, weight, bias, eps, out_dtype):
    return x.new_empty(x.shape, dtype=_dtype(out_dtype))


@torch.library.custom_op("mpk::add_layer_norm", mutates_args=())
def add_layer_norm(
    x: torch.Tensor, update: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, eps: float, out_dtype: int
) -> Tuple[torch.Tensor, torch.Tensor]:
    """``r = x + update`` (FP32) and ``LayerNorm(r)`` (``mpk_layernorm``)."""
    d = x.shape[-1]
    residual = torch.empty_like(x)
    out = torch.empty(x.shape, device=x.device, dtype=_dtype(out_dtype))
    _require_aligned("unsupported residual/LayerNorm inputs", x, update, weight, bias, residual, out)
    _lib.check(
        _lib.load().mpk_layernorm(
            x.data_ptr(), update.data_ptr(), weight.data_ptr(), bias.data_ptr(), residual.data_ptr(), out.data_ptr(),
            int(out_dtype), _rows(x, d), d, float(eps), _lib.stream_handle(x.device),
        ),
        "mpk_layernorm",
    )
    return residual, out


@add_layer_norm.register_fake
def _(x, update, weight, bias, eps, out_dtype):
    return torch.empty_like(x), x.new_empty(x.shape, dtype=_dtype(out_dtype))


# --------------------------------------------------------------------------- projections


@torch.library.custom_op("mpk::linear", mutates_args=())
def linear(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out_dtype: int, gelu: bool, variant: int
) -> torch.Tensor:
    """``act(fp16(x) W^T + b)`` (``mpk_linear``)."""
    n, k = weight.shape
    out = torch.empty((*x.shape[:-1], n), device=x.device, dtype=_dtype(out_dtype))
    _require_aligned("unsupported mixed projection inputs", x, weight, bias, out)
    _lib.check(
        _lib.load().mpk_linear(
            x.data_ptr(), _lib.dtype_code(x.dtype), weight.data_ptr(), bias.data_ptr(), out.data_ptr(),
            int(out_dtype), 1 if gelu else 0, _rows(x, k), n, k, int(variant), _lib.stream_handle(x.device),
        ),
        "mpk_linear",
    )
    return out


@linear.register_fake
def _(x, weight, bias, out_dtype, gelu, variant):
    return x.new_empty((*x.shape[:-1], weight.shape[0]), dtype=_dtype(out_dtype))


@torch.library.custom_op("mpk::linear_qscaled", mutates_args=())
def linear_qscaled(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, out_dtype: int, q_cols: int, q_scale: float,
    variant: int,
) -> torch.Tensor:
    """``fp16(x) W^T + b`` with columns below ``q_cols`` multiplied by ``q_scale`` before the
    output rounding (``mpk_linear_qscaled``)."""
    n, k = weight.shape
    out = torch.empty((*x.shape[:-1], n), device=x.device, dtype=_dtype(out_dtype))
    _require_aligned("unsupported mixed projection inputs", x, weight, bias, out)
    _lib.check(
        _lib.load().mpk_linear_qscaled(
            x.data_ptr(), _lib.dtype_code(x.dtype), weight.data_ptr(), bias.data_ptr(), out.data_ptr(),
            int(out_dtype), _rows(x, k), n, k, int(q_cols), float(q_scale), int(variant), _lib.stream_handle(x.device),
        ),
        "mpk_linear_qscaled",
    )
    return out


@linear_qscaled.register_fake
def _(x, weight, bias, out_dtype, q_cols, q_scale, variant):
    return x.new_empty((*x.shape[:-1], weight.shape[0]), dtype=_dtype(out_dtype))


def _launch_linear_residual(x, weight, bias, residual, out, variant) -> None:
    n, k = weight.shape
    _require_aligned("unsupported mixed projection/residual inputs", x, weight, bias, residual, out)
    _lib.check(
        _lib.load().mpk_linear_residual(
            x.data_ptr(), _lib.dtype_code(x.dtype), weight.data_ptr(), bias.data_ptr(), residual.data_ptr(),
            out.data_ptr(), _rows(x, k), n, k, int(variant), _lib.stream_handle(x.device),
        ),
        "mpk_linear_residual",
    )


@torch.library.custom_op("mpk::linear_residual", mutates_args=())
def linear_residual(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, residual: torch.Tensor, variant: int
) -> torch.Tensor:
    """``fp16(x) W^T + b + residual`` in FP32 (``mpk_linear_residual``)."""
    out = torch.empty_like(residual)
    _launch_linear_residual(x, weight, bias, residual, out, variant)
    return out


@linear_residual.register_fake
def _(x, weight, bias, residual, variant):
    return torch.empty_like(residual)


@torch.library.custom_op("mpk::linear_residual_into", mutates_args=("out",))
def linear_residual_into(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, residual: torch.Tensor, out: torch.Tensor, variant: int
) -> None:
    """As ``linear_residual`` into a caller-supplied FP32 ``out`` (which may be ``residual``)."""
    _launch_linear_residual(x, weight, bias, residual, out, variant)


@linear_residual_into.register_fake
def _(x, weight, bias, residual, out, variant):
    return None


@torch.library.custom_op("mpk::linear_residual_layer_norm", mutates_args=())
def linear_residual_layer_norm(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, residual: torch.Tensor, gamma: torch.Tensor,
    beta: torch.Tensor, eps: float, out_dtype: int, variant: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Square projection + residual + LayerNorm with whole rows per wave (``mpk_linear_residual_layernorm``)."""
    d = weight.shape[0]
    residual_out = torch.empty_like(residual)
    normalized = torch.empty(residual.shape, device=x.device, dtype=_dtype(out_dtype))
    _require_aligned("unsupported fused projection/residual/LayerNorm inputs", x, weight, bias, residual, gamma, beta,
                     residual_out, normalized)
    _lib.check(
        _lib.load().mpk_linear_residual_layernorm(
            x.data_ptr(), _lib.dtype_code(x.dtype), weight.data_ptr(), bias.data_ptr(), residual.data_ptr(),
            gamma.data_ptr(), beta.data_ptr(), residual_out.data_ptr(), normalized.data_ptr(), int(out_dtype),
            _rows(x, d), d, float(eps), int(variant), _lib.stream_handle(x.device),
        ),
        "mpk_linear_residual_layernorm",
    )
    return residual_out, normalized


@linear_residual_layer_norm.register_fake
def _(x, weight, bias, residual, gamma, beta, eps, out_dtype, variant):
    return torch.empty_like(residual), residual.new_empty(residual.shape, dtype=_dtype(out_dtype))


@torch.library.custom_op("mpk::linear_add_layer_norm", mutates_args=())
def linear_add_layer_norm(
    x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor, residual: torch.Tensor, gamma: torch.Tensor,
    beta: torch.Tensor, eps: float, out_dtype: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Projection (any input width) + residual + LayerNorm on large GEMM tiles (``mpk_linear_add_layernorm``)."""
    n, k = weight.shape
    residual_out = torch.empty_like(residual)
    normalized = torch.empty(residual.shape, device=x.device, dtype=_dtype(out_dtype))
    _require_aligned("unsupported projection/residual/LayerNorm inputs", x, weight, bias, residual, gamma, beta,
                     residual_out, normalized)
    _lib.check(
        _lib.load().mpk_linear_add_layernorm(
            x.data_ptr(), _lib.dtype_code(x.dtype), weight.data_ptr(), bias.data_ptr(), residual.data_ptr(),
            gamma.data_ptr(), beta.data_ptr(), residual_out.data_ptr(), normalized.data_ptr(), int(out_dtype),
            _rows(residual, n), n, k, float(eps), _lib.stream_handle(x.device),
        ),
        "mpk_linear_add_layernorm",
    )
    return residual_out, normalized


@linear_add_layer_norm.register_fake
def _(x, weight, bias, residual, gamma, beta, eps, out_dtype):
    return torch.empty_like(residual), residual.new_empty(residual.shape, dtype=_dtype(out_dtype))


@torch.library.custom_op("mpk::ffn_residual_layer_norm", mutates_args=())
def ffn_residual_layer_norm(
    x: torch.Tensor, w_in: torch.Tensor, b_in: torch.Tensor, w_out: torch.Tensor, b_out: torch.Tensor,
    residual: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float, out_dtype: int, variant: int,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Whole FFN (hidden on chip) + residual + LayerNorm (``mpk_ffn_residual_layernorm``)."""
    f, d = w_in.shape
    residual_out = torch.empty_like(residual)
    normalized = torch.empty(residual.shape, device=x.device, dtype=_dtype(out_dtype))
    _require_aligned("unsupported fused FFN inputs", x, w_in, b_in, w_out, b_out, residual, gamma, beta, residual_out,
                     normalized)
    _lib.check(
        _lib.load().mpk_ffn_residual_layernorm(
            x.data_ptr(), _lib.dtype_code(x.dtype), w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(),
            b_out.data_ptr(), residual.data_ptr(), gamma.data_ptr(), beta.data_ptr(), residual_out.data_ptr(),
            normalized.data_ptr(), int(out_dtype), _rows(x, d), d, f, float(eps), int(variant),
            _lib.stream_handle(x.device),
        ),
        "mpk_ffn_residual_layernorm",
    )
    return residual_out, normalized


@ffn_residual_layer_norm.register_fake
def _(x, w_in, b_in, w_out, b_out, residual, gamma, beta, eps, out_dtype, variant):
    return torch.empty_like(residual), residual.new_empty(residual.shape, dtype=_dtype(out_dtype))


@torch.library.custom_op("mpk::ffn_residual_layer_norm_into", mutates_args=("normalized",))
def ffn_residual_layer_norm_into(
    x: torch.Tensor, w_in: torch.Tensor, b_in: torch.Tensor, w_out: torch.Tensor, b_out: torch.Tensor,
    residual: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float, variant: int,
    normalized: torch.Tensor, store_residual: bool,
) -> torch.Tensor:
    """``ffn_residual_layer_norm`` with the normalized output written into ``normalized``
    (contiguous, residual's shape, FP32 or FP16: a caller's preallocated output slice, so
    no copy follows); returns the residual output, or an empty tensor when
    ``store_residual`` is false (the kernel then stores only the normalized output)."""
    f, d = w_in.shape
    residual_out = torch.empty_like(residual) if store_residual else residual.new_empty(0)
    _require_aligned("unsupported fused FFN inputs", x, w_in, b_in, w_out, b_out, residual, gamma, beta, residual_out,
                     normalized)
    _lib.check(
        _lib.load().mpk_ffn_residual_layernorm(
            x.data_ptr(), _lib.dtype_code(x.dtype), w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(),
            b_out.data_ptr(), residual.data_ptr(), gamma.data_ptr(), beta.data_ptr(),
            residual_out.data_ptr() if store_residual else None,
            normalized.data_ptr(), _lib.dtype_code(normalized.dtype), _rows(x, d), d, f, float(eps), int(variant),
            _lib.stream_handle(x.device),
        ),
        "mpk_ffn_residual_layernorm",
    )
    return residual_out


@ffn_residual_layer_norm_into.register_fake
def _(x, w_in, b_in, w_out, b_out, residual, gamma, beta, eps, variant, normalized, store_residual):
    return torch.empty_like(residual) if store_residual else residual.new_empty(0)


@torch.library.custom_op("mpk::ffn_residual_layer_norm_final", mutates_args=())
def ffn_residual_layer_norm_final(
    x: torch.Tensor, w_in: torch.Tensor, b_in: torch.Tensor, w_out: torch.Tensor, b_out: torch.Tensor,
    residual: torch.Tensor, gamma: torch.Tensor, beta: torch.Tensor, eps: float, out_dtype: int, variant: int,
) -> torch.Tensor:
    """``ffn_residual_layer_norm`` for a last layer: only the normalized output is stored and
    returned (the residual stream after it is not read)."""
    normalized = torch.empty(residual.shape, device=x.device, dtype=_dtype(out_dtype))
    ffn_residual_layer_norm_into(x, w_in, b_in, w_out, b_out, residual, gamma, beta, eps, variant, normalized, False)
    return normalized


@ffn_residual_layer_norm_final.register_fake
def _(x, w_in, b_in, w_out, b_out, residual, gamma, beta, eps, out_dtype, variant):
    return residual.new_empty(residual.shape, dtype=_dtype(out_dtype))


# --------------------------------------------------------------------------- attention


@torch.library.custom_op("mpk::attention", mutates_args=())
def attention(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_valid: Optional[torch.Tensor], scale: float, causal: bool,
    out_dtype: int, variant: int,
) -> torch.Tensor:
    """Flash attention over strided ``[B, H, S, hd]`` views -> contiguous ``[B, S, H, hd]``
    (``mpk_causal_attention``).  ``key_valid``: optional uint8 ``[B, S]``, nonzero = valid key."""
    batch, heads, seq_len, head_dim = q.shape
    _require_aligned(f"unsupported custom-attention input: shape={tuple(q.shape)}, dtype={q.dtype}", q, k, v)
    out = torch.empty((batch, seq_len, heads, head_dim), device=q.device, dtype=_dtype(out_dtype))
    o_strides = (out.stride(0), out.stride(2), out.stride(1), out.stride(3))
    _lib.check(
        _lib.load().mpk_causal_attention(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), _lib.dtype_code(q.dtype), int(out_dtype),
            _lib.strides4(q.stride()), _lib.strides4(k.stride()), _lib.strides4(v.stride()), _lib.strides4(o_strides),
            batch, heads, seq_len, head_dim, float(scale), 1 if causal else 0, _ptr(key_valid), int(variant),
            _lib.stream_handle(q.device),
        ),
        "mpk_causal_attention",
    )
    return out


@attention.register_fake
def _(q, k, v, key_valid, scale, causal, out_dtype, variant):
    batch, heads, seq_len, head_dim = q.shape
    return q.new_empty((batch, seq_len, heads, head_dim), dtype=_dtype(out_dtype))


@torch.library.custom_op("mpk::attention_prescaled", mutates_args=())
def attention_prescaled(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, key_valid: Optional[torch.Tensor], causal: bool,
    out_dtype: int, variant: int,
) -> torch.Tensor:
    """Flash attention over FP16 views whose q already holds q * scale * log2(e)
    (``mpk_causal_attention_prescaled``) -> contiguous ``[B, S, H, hd]``."""
    batch, heads, seq_len, head_dim = q.shape
    _require_aligned(f"unsupported custom-attention input: shape={tuple(q.shape)}, dtype={q.dtype}", q, k, v)
    out = torch.empty((batch, seq_len, heads, head_dim), device=q.device, dtype=_dtype(out_dtype))
    o_strides = (out.stride(0), out.stride(2), out.stride(1), out.stride(3))
    _lib.check(
        _lib.load().mpk_causal_attention_prescaled(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), int(out_dtype),
            _lib.strides4(q.stride()), _lib.strides4(k.stride()), _lib.strides4(v.stride()), _lib.strides4(o_strides),
            batch, heads, seq_len, head_dim, 1 if causal else 0, _ptr(key_valid), int(variant),
            _lib.stream_handle(q.device),
        ),
        "mpk_causal_attention_prescaled",
    )
    return out


@attention_prescaled.register_fake
def _(q, k, v, key_valid, causal, out_dtype, variant):
    batch, heads, seq_len, head_dim = q.shape
    return q.new_empty((batch, seq_len, heads, head_dim), dtype=_dtype(out_dtype))


# --------------------------------------------------------------------------- whole-layer fusions


@torch.library.custom_op("mpk::layer_norm_qkv", mutates_args=())
def layer_norm_qkv(
    x: torch.Tensor, ln_w: torch.Tensor, ln_b: torch.Tensor, w_qkv: torch.Tensor, b_qkv: torch.Tensor, eps: float,
    variant: int, q_scale: float = 0.0,
) -> torch.Tensor:
    """``fp16(LayerNorm(x)) W_qkv^T + b`` -> FP16 ``[..., 3D]`` (``mpk_layernorm_qkv``); with
    ``q_scale`` != 0 the q columns are multiplied by it before the FP16 rounding
    (``mpk_layernorm_qkv_qscaled``)."""
    d = x.shape[-1]
    out = torch.empty((*x.shape[:-1], 3 * d), device=x.device, dtype=torch.float16)
    _require_aligned("unsupported LayerNorm/QKV inputs", x, ln_w, ln_b, w_qkv, b_qkv, out)
    lib = _lib.load()
    args = (x.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(), w_qkv.data_ptr(), b_qkv.data_ptr(), out.data_ptr(),
            _rows(x, d), d, float(eps))
    tail = (int(variant), _lib.stream_handle(x.device))
    if q_scale:
        _lib.check(lib.mpk_layernorm_qkv_qscaled(*args, float(q_scale), *tail), "mpk_layernorm_qkv_qscaled")
    else:
        _lib.check(lib.mpk_layernorm_qkv(*args, *tail), "mpk_layernorm_qkv")
    return out


@layer_norm_qkv.register_fake
def _(x, ln_w, ln_b, w_qkv, b_qkv, eps, variant, q_scale=0.0):
    return x.new_empty((*x.shape[:-1], 3 * x.shape[-1]), dtype=torch.float16)


@torch.library.custom_op("mpk::layer_tail", mutates_args=())
def layer_tail(
    ctx: torch.Tensor, residual: torch.Tensor, tensors: List[torch.Tensor], w_qkv: Optional[torch.Tensor],
    b_qkv: Optional[torch.Tensor], ln2_eps: float, next_eps: float, variant: int, q_scale: float = 0.0,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Out-projection through the next layer's QKV (or the final LayerNorm) in one kernel (``mpk_layer_tail``).

    ``tensors`` = [w_o, b_o, ln2_w, ln2_b, w_in, b_in, w_out, b_out, next_ln_w, next_ln_b].
    Returns ``(residual_out, qkv FP16 [..., 3D])``, or ``(residual_out, normalized FP32)``
    when ``w_qkv`` is None (last layer).  ``q_scale`` != 0 multiplies the next q columns by it
    before the FP16 rounding (``mpk_layer_tail_qscaled``).
    """
    w_o, b_o, ln2_w, ln2_b, w_in, b_in, w_out, b_out, next_w, next_b = tensors
    d = ctx.shape[-1]
    f = w_in.shape[0]
    last = w_qkv is None
    residual_out = torch.empty_like(residual)
    shape = ctx.shape if last else (*ctx.shape[:-1], 3 * d)
    out = torch.empty(shape, device=ctx.device, dtype=torch.float32 if last else torch.float16)
    _require_aligned("unsupported fused layer-tail inputs", ctx, residual, *tensors, w_qkv, b_qkv, residual_out, out)
    lib = _lib.load()
    args = (ctx.data_ptr(), residual.data_ptr(), w_o.data_ptr(), b_o.data_ptr(), ln2_w.data_ptr(), ln2_b.data_ptr(),
            w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(), b_out.data_ptr(), next_w.data_ptr(),
            next_b.data_ptr(), _ptr(w_qkv), _ptr(b_qkv), residual_out.data_ptr(), out.data_ptr(), 1 if last else 0,
            _rows(ctx, d), d, f, float(ln2_eps), float(next_eps))
    tail = (int(variant), _lib.stream_handle(ctx.device))
    if q_scale:
        _lib.check(lib.mpk_layer_tail_qscaled(*args, float(q_scale), *tail), "mpk_layer_tail_qscaled")
    else:
        _lib.check(lib.mpk_layer_tail(*args, *tail), "mpk_layer_tail")
    return residual_out, out


@layer_tail.register_fake
def _(ctx, residual, tensors, w_qkv, b_qkv, ln2_eps, next_eps, variant, q_scale=0.0):
    d = ctx.shape[-1]
    if w_qkv is None:
        return torch.empty_like(residual), ctx.new_empty(ctx.shape, dtype=torch.float32)
    return torch.empty_like(residual), ctx.new_empty((*ctx.shape[:-1], 3 * d), dtype=torch.float16)


@torch.library.custom_op("mpk::attention_layer_tail", mutates_args=())
def attention_layer_tail(
    qkv: torch.Tensor, residual: torch.Tensor, tensors: List[torch.Tensor], w_qkv: Optional[torch.Tensor],
    b_qkv: Optional[torch.Tensor], heads: int, scale: float, causal: bool, ln2_eps: float, next_eps: float,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Attention (head dim 32) from this layer's packed ``qkv [B, S, 3D]`` through the next
    layer's QKV (or the final LayerNorm) in one kernel (``mpk_attention_layer_tail``).

    ``tensors`` as for ``layer_tail``.  Returns ``(residual_out, next qkv FP16 [B, S, 3D])``,
    or ``(residual_out, normalized FP32)`` when ``w_qkv`` is None (last layer); the next
    layer's QKV is always a new tensor (the kernel reads ``qkv`` while it writes it).
    """
    w_o, b_o, ln2_w, ln2_b, w_in, b_in, w_out, b_out, next_w, next_b = tensors
    d = residual.shape[-1]
    f = w_in.shape[0]
    last = w_qkv is None
    residual_out = torch.empty_like(residual)
    shape = residual.shape if last else (*residual.shape[:-1], 3 * d)
    out = torch.empty(shape, device=qkv.device, dtype=torch.float32 if last else torch.float16)
    _require_aligned("unsupported fused attention layer-tail inputs", qkv, residual, *tensors, w_qkv, b_qkv,
                     residual_out, out)
    _lib.check(
        _lib.load().mpk_attention_layer_tail(
            qkv.data_ptr(), residual.data_ptr(), w_o.data_ptr(), b_o.data_ptr(), ln2_w.data_ptr(),
            ln2_b.data_ptr(), w_in.data_ptr(), b_in.data_ptr(), w_out.data_ptr(), b_out.data_ptr(),
            next_w.data_ptr(), next_b.data_ptr(), _ptr(w_qkv), _ptr(b_qkv), residual_out.data_ptr(),
            out.data_ptr(), 1 if last else 0, _rows(residual, d), d, f, int(heads), int(residual.shape[-2]),
            float(scale), 1 if causal else 0, float(ln2_eps), float(next_eps), _lib.stream_handle(qkv.device),
        ),
        "mpk_attention_layer_tail",
    )
    return residual_out, out


@attention_layer_tail.register_fake
def _(qkv, residual, tensors, w_qkv, b_qkv, heads, scale, causal, ln2_eps, next_eps):
    d = residual.shape[-1]
    if w_qkv is None:
        return torch.empty_like(residual), residual.new_empty(residual.shape, dtype=torch.float32)
    return torch.empty_like(residual), residual.new_empty((*residual.shape[:-1], 3 * d), dtype=torch.float16)
