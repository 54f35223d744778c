"""MI355X-native mixed-precision causal-Transformer forward.

Hand-written gfx950 HIP kernels (``csrc/``) behind the C ABI declared in
``include/mpk.h`` (built into ``libmpk.so`` by ``build.py``), with Python
operators and modules that keep the reference project's ``mixed_precision``
and ``custom_kernel`` interfaces.
"""

from .config import BENCHMARK_CONFIGS, TransformerConfig

__all__ = ["BENCHMARK_CONFIGS", "TransformerConfig"]
