"""Causal flash attention on gfx950 (replaces the reference's custom_kernel Triton attention)."""

from .hip_attention import (
    attention,
    causal_attention,
    fp16_causal_attention,
    is_fp16_supported,
    is_supported,
    launch_causal_attention,
)

__all__ = [
    "attention",
    "causal_attention",
    "fp16_causal_attention",
    "is_fp16_supported",
    "is_supported",
    "launch_causal_attention",
]
