"""Mixed FP16/FP32 Transformer candidate on gfx950 HIP kernels (drop-in for the reference's package)."""

from .transformer import MixedPrecisionTransformer, copy_mixed_model_weights

__all__ = ["MixedPrecisionTransformer", "copy_mixed_model_weights"]
