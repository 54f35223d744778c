"""Shape-dispatch table for the HIP forward (replaces the reference's exact-shape route flags).

The reference selects Triton routes with hard-coded exact-shape booleans
(``mixed_precision/transformer.py:337-448``) and per-row-count tile tables
(``:88-99, :198-205, :518-560``); any shape outside them falls back to vendor
ops.  Here every supported shape takes the same HIP route; what varies with
the shape is only

* which fusions apply.  Up to d_model 128 the out-projection and the FFN
  run as row-owning kernels with the residual add and LayerNorm in the
  epilogue (``LN_FUSED_WIDTHS`` bounds what those kernels accept).  Wider
  models (``WIDE_GEMM_FROM``) and disabled fusions run the projections as
  large-tile GEMMs with the bias/GELU/residual add in the epilogue and a
  separate LayerNorm: a row-owning kernel would re-read a D x D (or D x F)
  weight for every 64-128 rows, while the GEMM tiles read it once per 256
  rows and keep the matrix cores busy, and
* the kernel tile variant of each launch.  Variant 0 defers to the
  library's built-in table (``mpk_*_auto_variant``), which holds the choices
  measured on MI355X (256 CUs, 64-lane waves); a ``Route`` can pin a variant
  per launch (tests and sweeps do).

At d_model 256 and 512 (``WIDE_LN_EPILOGUE_WIDTHS``) the GEMM route's
out-projection carries the next LayerNorm in its epilogue (``wide_ln_epilogue``):
a 256 x 256 (d 256) or 128 x 512 (d 512) output tile holds whole rows, so the row
statistics are exchanged across its waves in LDS and no separate LayerNorm launch
re-reads the residual stream.  The FFN-output projection does the same at d_model
256 (``wide_ln_ffn_out``); at 512 its K = ffn_dim loop runs faster on 256 x 256
tiles with 64-wide K chunks than on the LDS-limited 128 x 512 LayerNorm tile
(32-wide chunks: 142 vs 113 us with the separate LayerNorm at cfg4), so it keeps
the separate LayerNorm there.

At d_model 256 the FFN runs as one kernel too (``WIDE_FFN_WIDTH``,
``fuse_full_ffn``): both products on 32x32 MFMAs with the hidden activation in
registers, the residual add and the next LayerNorm in its epilogue, so that
route launches, per layer, the QKV projection, attention, the out-projection
(+ residual + LayerNorm) and the FFN (+ residual + LayerNorm).

When the whole layer tail fits one kernel (``LAYER_TAIL_SHAPES``) the forward
runs 1 + 2L launches: LayerNorm+QKV, then per layer attention and the fused
tail (out-proj+LN2+FFN+LN1'+QKV', or the final LayerNorm on the last layer).

Tile variants (the library's tables, ``mpk_*_auto_variant``, pick among them; see the
kernel sources for the exact tiles):
  projections (mpk_linear, mpk_linear_residual)
                           1: 128x128 (2x2 waves)  2: 128x64  3: 128x32  4: 64x128
                           5: 256x128 double-buffered  6: 256x128 single-buffered
                           7: 256x256 persistent tiles, 8 waves of 128x64, operands
                              through registers into LDS
                           8: as 7 with LDS-DMA operand staging (four-stage ring; FP16 X,
                              K % 32 == 0, K >= 128; others run 7) - the wide-model choice
                           9: X-stationary 256-token tiles, W streamed in 64-row blocks (FP16
                              X, K = 128 / 256, N % 64 == 0, bias or GELU epilogue; others run
                              8) - the choice for those K from 65,536 rows
  out-proj + LN (mpk_linear_residual_layernorm)
                           1: 64 rows/WG           2: 128 rows/WG (row-owning waves, d <= 128)
                           3: GEMM tiles holding whole rows with a cross-wave LayerNorm
                              (d 256: 256x256 tiles, 64-wide K chunks; d 512: 128x512, 32-wide)
  row-wide LayerNorm GEMM (mpk_linear_add_layernorm, d 256 / 512, any K): the variant-3 tiles
  fused FFN + LN           1: 16 rows/wave         2: 32 rows/wave (d <= 256)
                           3: wide kernel, one wave per SIMD (d = 256, FP16 input)
                           4: role-split wide kernel, a vector and a matrix wave per SIMD
                              (d = 256) - the built-in choice at d 256
  attention                16x16-MFMA kernel: 1: 16 queries/wave, 64-key tiles, 4 waves
                           2: 32 q/wave  3: 32 q/wave, 128-key tiles  4: 32 q/wave, 8 waves
                           5: 16 q/wave, 128-key tiles
                           32x32-MFMA kernel (hd 32 and 64, 32 queries/wave):
                           6: 64-key tiles, 4 waves  7: 64-key tiles, 8 waves
                           8: 128-key tiles, 4 waves
  layer tail / LN+QKV      1: 8 waves x 16 rows    2: 8 waves x 32 rows
                           3: 4 waves x 16 rows (when 128-row tiles would leave CUs idle)
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Tuple

import torch

LN_FUSED_WIDTHS = (32, 64, 128, 256, 512)
ATTENTION_HEAD_DIMS = (8, 16, 32, 64, 128, 256)
# (d_model, ffn_dim) pairs built into the whole-layer tail kernel (its weights fit in LDS);
# must equal mpk_layer_tail_supported / mpk_layernorm_qkv_supported in the library.
LAYER_TAIL_SHAPES = frozenset({(32, 32), (32, 64), (32, 128), (64, 64), (64, 128), (64, 256), (128, 128)})
LAYERNORM_QKV_WIDTHS = frozenset({32, 64, 128})
# Attention inside the layer-tail kernel: one launch per layer for short sequences made of
# whole 64-row tiles, without a key mask.  Head dim 32 on every tail shape, head dim 16 on
# d_model 32 and 64 (attention_tail_supported must equal mpk_attention_layer_tail_supported).
ATTENTION_TAIL_ROWS = 64
# Where the route uses it: the longest sequence per (d_model, head dim), from whole forwards
# timed fused vs separate attention + tail (HIP-graph replay on MI355X, one process):
#   d_model 32, hd 32: -18 to -20 % at 128 and 256 positions
#   d_model 64, hd 32: -10 to -17 % at 128 and 256; +40 % at 512 (a workgroup's 64 rows then
#                      walk 8 key tiles with one wave per SIMD, where the attention kernel
#                      spreads them over many CUs)
#   d_model 32, hd 16: -10 to -13 % at 128, -6 to -10 % at 256 (cfg3), -3 to -5 % at 512
#   d_model 64, hd 16: -6 to -9 % at 128; +4 to +9 % at 256
#   d_model 128, hd 32: slower at every length (+2-4 % at 128 positions: its register-resident
#                      QKV weights and four heads' softmax state exceed the VGPRs)
ATTENTION_TAIL_ROUTE_MAX_SEQ = {(32, 32): 256, (64, 32): 256, (32, 16): 512, (64, 16): 128}


def attention_tail_supported(d_model: int, ffn_dim: int, heads: int) -> bool:
    """Shapes built into the fused attention + layer-tail kernel (``mpk_attention_layer_tail_supported``)."""
    d, f, h = int(d_model), int(ffn_dim), int(heads)
    if (d, f) not in LAYER_TAIL_SHAPES or h <= 0 or d % h:
        return False
    hd = d // h
    return hd == 32 or (hd == 16 and d <= 64)
# From this width up the out-projection and FFN run as GEMMs + a separate LayerNorm.
WIDE_GEMM_FROM = 256
# GEMM-route widths whose out-projection fuses the next LayerNorm (tiles holding whole
# rows); must equal the widths mpk_linear_add_layernorm accepts.  The FFN-output
# projection fuses it at the widths of WIDE_LN_FFN_OUT_WIDTHS.
WIDE_LN_EPILOGUE_WIDTHS = (256, 512)
WIDE_LN_FFN_OUT_WIDTHS = (256,)
# Width of the wide fused FFN kernel (32x32-MFMA, hidden on chip) and its largest ffn_dim;
# must equal ffn_wide_supported in the library.
WIDE_FFN_WIDTH = 256
WIDE_FFN_MAX_F = 8192


@dataclass(frozen=True)
class Route:
    """Everything the forward needs to know about how to run one configuration."""

    supported: bool
    reason: str
    normalized_dtype: torch.dtype = torch.float16
    fp16_attention: bool = True
    fuse_attention_output_norm: bool = True
    fuse_full_ffn: bool = True
    fuse_layer_tail: bool = False
    fuse_attention_tail: bool = False  # attention inside the layer tail, up to attention_tail_max_seq positions
    attention_tail_max_seq: int = 0
    # head dim 32: from 256 keys the QKV producer (projection, layer tail or LayerNorm + QKV)
    # folds the attention scale into q and the 32x32 attention kernel skips its per-score FMA
    # (prescaled_attention_for; not where attention runs inside the layer tail)
    prescale_q: bool = False
    wide_ln_epilogue: bool = False
    wide_ln_ffn_out: bool = False
    qkv_variant: int = 0
    attention_variant: int = 0
    out_ln_variant: int = 0
    ffn_variant: int = 0
    ffn_in_variant: int = 0
    ffn_out_variant: int = 0
    out_proj_variant: int = 0
    tail_variant: int = 0
    head_variant: int = 0
    notes: Tuple[str, ...] = field(default_factory=tuple)

    def describe(self) -> Dict[str, object]:
        return {
            "supported": self.supported,
            "reason": self.reason,
            "normalized_stream": "fp16" if self.normalized_dtype == torch.float16 else "fp32",
            "attention": "hip_fp16_flash" if self.fp16_attention else "hip_fp32io_flash",
            "attention_output_norm_fusion": self.fuse_attention_output_norm,
            "full_ffn_fusion": self.fuse_full_ffn,
            "layer_tail_fusion": self.fuse_layer_tail,
            "attention_in_layer_tail": self.fuse_attention_tail,
            "wide_ln_epilogue": self.wide_ln_epilogue,
            "wide_ln_ffn_out": self.wide_ln_ffn_out,
            "variants": {
                "qkv": self.qkv_variant,
                "attention": self.attention_variant,
                "out_ln": self.out_ln_variant,
                "ffn": self.ffn_variant,
                "ffn_in": self.ffn_in_variant,
                "ffn_out": self.ffn_out_variant,
                "out_proj": self.out_proj_variant,
                "layer_tail": self.tail_variant,
                "layernorm_qkv": self.head_variant,
            },
        }


def plan(
    config,
    *,
    enable_attention_output_norm_fusion: bool = True,
    enable_full_ffn_fusion: bool = True,
    enable_fp16_custom_attention: bool = True,
    enable_fp16_normalized_stream: bool = True,
) -> Route:
    """Return the route for ``config`` (any object with the TransformerConfig fields)."""
    d = int(config.d_model)
    f = int(config.ffn_dim)
    h = int(config.num_heads)
    if h <= 0 or d % h != 0:
        return Route(False, "d_model must be divisible by num_heads")
    hd = d // h
    if hd not in ATTENTION_HEAD_DIMS:
        return Route(False, f"head_dim {hd} not in {ATTENTION_HEAD_DIMS}")
    if d % 8 != 0 or f % 8 != 0:
        return Route(False, "d_model and ffn_dim must be multiples of 8")
    if d > 2048:
        return Route(False, "d_model above 2048")
    narrow = d in LN_FUSED_WIDTHS and d < WIDE_GEMM_FROM
    fuse_out = enable_attention_output_norm_fusion and narrow
    wide_ffn = d == WIDE_FFN_WIDTH and f <= WIDE_FFN_MAX_F
    fuse_ffn = enable_full_ffn_fusion and (narrow or wide_ffn) and f % 32 == 0
    # The layer-tail kernel chains out-proj+LN2 -> FFN+LN -> next QKV; it needs both
    # fusions, the FP16 normalized stream and FP16 attention I/O.
    fuse_tail = (
        fuse_out and fuse_ffn and enable_fp16_normalized_stream and enable_fp16_custom_attention
        and (d, f) in LAYER_TAIL_SHAPES and d in LAYERNORM_QKV_WIDTHS
    )
    wide_ln = (
        enable_attention_output_norm_fusion and enable_full_ffn_fusion and not narrow
        and d in WIDE_LN_EPILOGUE_WIDTHS
    )
    attn_tail_max_seq = (
        ATTENTION_TAIL_ROUTE_MAX_SEQ.get((d, hd), 0) if fuse_tail and attention_tail_supported(d, f, h) else 0
    )
    fuse_attn_tail = attn_tail_max_seq > 0
    route = Route(
        True,
        "hip",
        normalized_dtype=torch.float16 if enable_fp16_normalized_stream else torch.float32,
        fp16_attention=enable_fp16_custom_attention,
        fuse_attention_output_norm=fuse_out,
        fuse_full_ffn=fuse_ffn,
        fuse_layer_tail=fuse_tail,
        fuse_attention_tail=fuse_attn_tail,
        attention_tail_max_seq=attn_tail_max_seq,
        prescale_q=enable_fp16_custom_attention and hd == 32,
        wide_ln_epilogue=wide_ln,
        wide_ln_ffn_out=wide_ln and d in WIDE_LN_FFN_OUT_WIDTHS,
    )
    return route


def attention_tail_for(route: Route, seq_len: int, masked: bool) -> bool:
    """Whether a forward over ``seq_len`` positions runs attention inside the layer-tail kernel:
    the route allows it (a supported shape listed in ATTENTION_TAIL_ROUTE_MAX_SEQ), no key
    mask, and the sequence is whole 64-row tiles of at most ``route.attention_tail_max_seq``
    positions."""
    return (
        route.fuse_attention_tail and not masked and 0 < seq_len <= route.attention_tail_max_seq
        and seq_len % ATTENTION_TAIL_ROWS == 0
    )


# Sequence length from which the built-in attention choice at head dim 32 is the 32x32 kernel
# (mpk_attention_auto_variant), whose steady tiles the pre-scaled q makes cheaper.
PRESCALED_ATTENTION_MIN_SEQ = 256


def prescaled_attention_for(route: Route, seq_len: int) -> bool:
    """Whether a forward over ``seq_len`` positions projects q pre-multiplied by the attention's
    scale * log2(e) and runs ``attention_prescaled`` as a launch of its own (the layer-tail route
    checks ``attention_tail_for`` first: attention inside the tail keeps its scaling).  Measured
    on MI355X in one process: attention at cfg5's shape 831 -> 764 us, at cfg2's 36 -> 34 us,
    from the per-score FMA it no longer needs."""
    return (
        route.prescale_q and seq_len >= PRESCALED_ATTENTION_MIN_SEQ and route.attention_variant in (0, 6, 7, 8)
    )
