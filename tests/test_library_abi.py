"""The C-ABI library: builds, loads, exports every symbol ``include/mpk.h`` declares, and
rejects bad arguments on the host before any launch (CPU only: no kernel runs)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from tiktoktechjam2026_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "mpk.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mpk_\w+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for required in (
        "mpk_layernorm",
        "mpk_linear",
        "mpk_linear_residual_layernorm",
        "mpk_ffn_residual_layernorm",
        "mpk_causal_attention",
        "mpk_status_string",
    ):
        assert required in names


def test_library_exports_every_declared_symbol(built_library):
    for name in declared_functions():
        assert hasattr(built_library, name), f"libmpk.so does not export {name}"
        assert name in _lib.SIGNATURES, f"_lib.SIGNATURES lacks {name}"
    assert built_library.mpk_version() >= 1


def test_status_strings(built_library):
    for code in (_lib.MPK_OK, _lib.MPK_EINVAL, _lib.MPK_EUNSUPPORTED, _lib.MPK_EALIGN):
        assert built_library.mpk_status_string(code)


def test_host_side_argument_rejection(built_library):
    lib = built_library
    null = None
    fake = ctypes.c_void_p(64)  # never dereferenced: every call below fails validation first
    assert lib.mpk_linear(null, 1, fake, fake, fake, 1, 0, 10, 16, 16, 0, null) == _lib.MPK_EINVAL
    assert lib.mpk_linear(fake, 7, fake, fake, fake, 1, 0, 10, 16, 16, 0, null) == _lib.MPK_EINVAL
    assert lib.mpk_linear(fake, 1, fake, fake, fake, 1, 0, 10, 12, 16, 0, null) == _lib.MPK_EUNSUPPORTED
    assert lib.mpk_linear(ctypes.c_void_p(72), 1, fake, fake, fake, 1, 0, 10, 16, 16, 0, null) == _lib.MPK_EALIGN
    assert lib.mpk_linear(fake, 1, fake, fake, fake, 1, 0, 10, 16, 16, 10, null) == _lib.MPK_EUNSUPPORTED
    assert lib.mpk_linear_residual(fake, 1, fake, fake, null, fake, 10, 16, 16, 0, null) == _lib.MPK_EINVAL
    assert lib.mpk_linear_residual(fake, 1, fake, fake, fake, fake, 10, 20, 16, 0, null) == _lib.MPK_EUNSUPPORTED
    assert lib.mpk_linear_residual(fake, 1, fake, fake, ctypes.c_void_p(72), fake, 10, 16, 16, 0, null) == _lib.MPK_EALIGN
    assert (
        lib.mpk_linear_residual_layernorm(fake, 1, fake, fake, fake, fake, fake, fake, fake, 1, 10, 96, 1e-5, 0, null)
        == _lib.MPK_EUNSUPPORTED
    )
    # the wide LayerNorm-epilogue GEMM takes n == 256 only, k % 8 == 0
    assert (
        lib.mpk_linear_add_layernorm(fake, 1, fake, fake, fake, fake, fake, fake, fake, 1, 10, 128, 256, 1e-5, null)
        == _lib.MPK_EUNSUPPORTED
    )
    assert (
        lib.mpk_linear_add_layernorm(fake, 1, fake, fake, fake, fake, fake, fake, fake, 1, 10, 256, 100, 1e-5, null)
        == _lib.MPK_EUNSUPPORTED
    )
    assert (
        lib.mpk_linear_add_layernorm(fake, 1, fake, fake, null, fake, fake, fake, fake, 1, 10, 256, 256, 1e-5, null)
        == _lib.MPK_EINVAL
    )
    assert (
        lib.mpk_linear_residual_layernorm(fake, 1, fake, fake, fake, fake, fake, fake, fake, 1, 10, 128, 1e-5, 3, null)
        == _lib.MPK_EUNSUPPORTED
    )
    assert (
        lib.mpk_ffn_residual_layernorm(
            fake, 1, fake, fake, fake, fake, fake, fake, fake, fake, fake, 1, 10, 128, 100, 1e-5, 0, null
        )
        == _lib.MPK_EUNSUPPORTED
    )
    assert lib.mpk_layernorm(fake, null, fake, fake, null, fake, 1, 10, 30, 1e-5, null) == _lib.MPK_EUNSUPPORTED
    assert lib.mpk_layernorm(fake, fake, fake, fake, null, fake, 1, 10, 32, 1e-5, null) == _lib.MPK_EINVAL
    s = _lib.strides4([1 << 20, 256, 1024, 1])
    assert (
        lib.mpk_causal_attention(fake, fake, fake, fake, 1, 1, s, s, s, s, 1, 1, 16, 24, 1.0, 1, null, 0, null)
        == _lib.MPK_EUNSUPPORTED
    )
    bad = _lib.strides4([1 << 20, 256, 1024, 2])
    assert (
        lib.mpk_causal_attention(fake, fake, fake, fake, 1, 1, bad, s, s, s, 1, 1, 16, 32, 1.0, 1, null, 0, null)
        == _lib.MPK_EUNSUPPORTED
    )


def test_auto_variant_queries(built_library):
    lib = built_library
    # the X-stationary tiles for K = 128 / 256 from 256 workgroup tiles (65,536 rows) on
    assert lib.mpk_linear_auto_variant(65536, 384, 128) == 9
    assert lib.mpk_linear_auto_variant(262144, 768, 256) == 9
    assert lib.mpk_linear_auto_variant(65535, 768, 256) == 8
    assert lib.mpk_linear_auto_variant(65536, 320, 256) in (1, 2, 3, 4)  # N / 64 < K / 32
    assert lib.mpk_linear_auto_variant(32768, 1536, 512) == 8
    assert lib.mpk_linear_residual_layernorm_auto_variant(65536, 128) in (1, 2)
    assert lib.mpk_linear_residual_layernorm_auto_variant(262144, 256) == 3
    assert lib.mpk_ffn_residual_layernorm_auto_variant(65536, 128, 128) in (1, 2)
    assert lib.mpk_attention_auto_variant(64, 4, 1024, 32) in range(1, 9)
    # short sequences stay on the 16x16 kernel; from 256 keys hd 32 / 64 use the 32x32 one
    assert lib.mpk_attention_auto_variant(64, 4, 128, 32) == 1
    assert lib.mpk_attention_auto_variant(64, 4, 256, 32) == 6
    assert lib.mpk_attention_auto_variant(64, 4, 256, 64) == 7
    assert lib.mpk_attention_auto_variant(16, 8, 2048, 64) == 6
    # the 32x32 kernel variants (6..8) only for head_dim 32 / 64
    for hd in (8, 16, 128, 256):
        for s in (128, 1024, 4096):
            assert lib.mpk_attention_auto_variant(4, 4, s, hd) in range(1, 6)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load()
