"""Per-kernel parity: each HIP kernel (through the C ABI wrappers) against a float64
CPU restatement of the same op on the same FP16-rounded operands.

Tolerances are stated per test; they bound FP32 accumulation-order differences
and, where an intermediate is rounded to FP16 inside the kernel, one FP16 ulp
of that intermediate.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _linear(in_f, out_f, device, seed):
    torch.manual_seed(seed)
    lin = nn.Linear(in_f, out_f)
    with torch.no_grad():
        lin.bias.uniform_(-0.5, 0.5)
    return lin.half().to(device)


def _norm(width, device, seed):
    g = torch.Generator().manual_seed(seed)
    norm = nn.LayerNorm(width)
    with torch.no_grad():
        norm.weight.copy_(1.0 + 0.1 * torch.randn(width, generator=g))
        norm.bias.copy_(0.1 * torch.randn(width, generator=g))
    return norm.to(device)


def _randn(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g) * scale


def _ln64(r, norm):
    w = norm.weight.detach().cpu().double()
    b = norm.bias.detach().cpu().double()
    mean = r.mean(-1, keepdim=True)
    var = ((r - mean) ** 2).mean(-1, keepdim=True)
    return (r - mean) / torch.sqrt(var + norm.eps) * w + b


def _close(actual, expected, atol, rtol, what):
    actual = actual.detach().cpu().double()
    expected = expected.double()
    err = (actual - expected).abs()
    bound = atol + rtol * expected.abs()
    bad = int((err > bound).sum())
    assert torch.isfinite(actual).all(), f"{what}: non-finite output"
    assert bad == 0, f"{what}: {bad} elements out of tolerance, max_err={float(err.max()):.3g}"


# --------------------------------------------------------------------------- LayerNorm


@pytest.mark.parametrize("width", [32, 96, 128, 256, 512, 1024])
@pytest.mark.parametrize("rows", [1, 37, 4099])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
def test_residual_layernorm(hip_device, width, rows, out_dtype):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import layer_norm, mixed_add_layer_norm

    x = _randn((rows, width), 1, 3.0)
    u = _randn((rows, width), 2)
    norm = _norm(width, hip_device, 3)
    res, out = mixed_add_layer_norm(x.to(hip_device), u.to(hip_device), norm, normalized_dtype=out_dtype)
    r64 = x.double() + u.double()
    _close(res, r64, 0.0, 1e-7, "residual")
    ref = _ln64(r64, norm)
    tol = 2e-5 if out_dtype == torch.float32 else 2 ** -10
    _close(out, ref, tol, tol, "normalized")
    plain = layer_norm(x.to(hip_device), norm, normalized_dtype=out_dtype)
    _close(plain, _ln64(x.double(), norm), tol, tol, "plain LN")


def test_layernorm_rejects_bad_inputs(hip_device):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_add_layer_norm

    norm = _norm(128, hip_device, 0)
    x = torch.zeros(4, 128, device=hip_device)
    with pytest.raises(ValueError):
        mixed_add_layer_norm(x.half(), x, norm, normalized_dtype=torch.float16)
    with pytest.raises(ValueError):
        mixed_add_layer_norm(x.cpu(), x.cpu(), norm, normalized_dtype=torch.float16)
    with pytest.raises(ValueError):
        mixed_add_layer_norm(x, x[:, :64].contiguous(), norm, normalized_dtype=torch.float16)


# --------------------------------------------------------------------------- projections


def _ref_linear(x, lin, gelu):
    xh = x.detach().cpu().half().double()
    w = lin.weight.detach().cpu().double()
    b = lin.bias.detach().cpu().double()
    y = xh @ w.t() + b
    if gelu:
        y = 0.5 * y * (1.0 + torch.erf(y / math.sqrt(2.0)))
    return y


@pytest.mark.parametrize(
    "m,n,k",
    [(8192, 384, 128), (1000, 96, 32), (333, 2048, 512), (5, 64, 64), (4096, 128, 128), (130, 768, 256),
     (257, 40, 24)],
)
@pytest.mark.parametrize("variant", [0, 1, 2, 3, 4, 5, 6, 7, 8])
def test_mixed_linear(hip_device, m, n, k, variant):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear

    lin = _linear(k, n, hip_device, 7)
    x32 = _randn((m, k), 11)
    for in_dtype in (torch.float32, torch.float16):
        for out_dtype in (torch.float32, torch.float16):
            for gelu in (False, True):
                x = x32.to(hip_device, in_dtype)
                y = mixed_linear(x, lin, output_dtype=out_dtype, fuse_gelu=gelu, variant=variant)
                assert y.dtype == out_dtype and y.shape == (m, n)
                ref = _ref_linear(x32, lin, gelu)
                tol = 1e-5 * math.sqrt(k) if out_dtype == torch.float32 else 2 ** -10
                _close(y, ref, tol, tol, f"linear in={in_dtype} out={out_dtype} gelu={gelu}")


@pytest.mark.parametrize(
    "m,n,k", [(8192, 384, 128), (333, 2048, 512), (1000, 200, 192), (130, 768, 256), (70000, 768, 256)]
)
def test_linear_large_tile_variants_bit_identical(hip_device, m, n, k):
    """Variants 7 (register staging) and 8 (LDS-DMA staging) accumulate the same MFMAs
    in the same order: identical outputs, including ragged tiles in M and N."""
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear

    print(f"\n[linear 7/8] m={m} n={n} k={k}", flush=True)
    lin = _linear(k, n, hip_device, 29)
    x = _randn((m, k), 31).to(hip_device, torch.float16)
    for out_dtype in (torch.float32, torch.float16):
        for gelu in (False, True):
            y7, y8 = (mixed_linear(x, lin, output_dtype=out_dtype, fuse_gelu=gelu, variant=v) for v in (7, 8))
            assert torch.equal(y7, y8), f"out={out_dtype} gelu={gelu}"


@pytest.mark.parametrize(
    "m,n,k",
    [(70000, 768, 256), (1, 768, 256), (255, 512, 256), (257, 384, 128), (3000, 256, 128), (4113, 1024, 256),
     (262244, 768, 256)],
)
def test_linear_x_stationary_variant_bit_identical(hip_device, m, n, k):
    """Variant 9 (X rows in registers, W streamed in 64-row blocks) accumulates the same
    MFMAs in the same order as variant 8: identical outputs for ragged M, tiles per workgroup
    from 1 to 5, N / 64 equal to and above K / 32, both epilogues, the q-scaled form, and
    FP16 / FP32 outputs."""
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear, mixed_linear_q_scaled

    print(f"\n[linear 8/9] m={m} n={n} k={k}", flush=True)
    lin = _linear(k, n, hip_device, 37)
    x = _randn((m, k), 41).to(hip_device, torch.float16)
    combos = [(torch.float16, False)] if m > 100000 else [(o, g) for o in (torch.float32, torch.float16) for g in (False, True)]
    for out_dtype, gelu in combos:
        y8, y9 = (mixed_linear(x, lin, output_dtype=out_dtype, fuse_gelu=gelu, variant=v) for v in (8, 9))
        assert torch.equal(y8, y9), f"out={out_dtype} gelu={gelu}"
    q8, q9 = (mixed_linear_q_scaled(x, lin, k, 0.25503486, variant=v) for v in (8, 9))
    assert torch.equal(q8, q9)
    plain = mixed_linear(x, lin, output_dtype=torch.float32, variant=9)
    _close(plain[:64], _ref_linear(x[:64], lin, False), 1e-5 * math.sqrt(k), 1e-5 * math.sqrt(k),
           "variant 9 against the float64 reference")


@pytest.mark.parametrize("n,variant", [(8, 0), (256, 7), (128, 1)])
def test_gelu_epilogue_accuracy(hip_device, n, variant):
    """The GEMM's GELU alone: X = [v, 0, ...] and W[:, 0] = 1 make every pre-activation
    exactly the FP16 value v, so the FP32 output is the kernel's GELU(v).  Every FP16 value
    in [-16, 16] plus large magnitudes, against float64 exact-erf GELU."""
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear

    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    v = bits.view(torch.float16)
    v = v[torch.isfinite(v) & (v.abs() <= 16)]
    v = torch.cat([v, torch.tensor([-65504.0, -100.0, -30.0, -20.0, 20.0, 30.0, 100.0, 65504.0]).half()])
    k = 8
    x = torch.zeros(v.numel(), k, dtype=torch.float16)
    x[:, 0] = v
    lin = torch.nn.Linear(k, n).to(hip_device).half()
    with torch.no_grad():
        lin.weight.zero_()
        lin.weight[:, 0] = 1.0
        lin.bias.zero_()
    y = mixed_linear(x.to(hip_device), lin, output_dtype=torch.float32, fuse_gelu=True, variant=variant).detach()
    vd = v.double()
    ref = 0.5 * vd * (1.0 + torch.erf(vd / math.sqrt(2.0)))
    err = (y.cpu().double() - ref[:, None]).abs()
    assert torch.isfinite(y).all()
    # A&S 7.1.26 erf (|error| <= 1.5e-7) plus FP32 rounding: below 1e-6 absolute where
    # |GELU| < 1 and 1e-6 relative above
    scaled = err / ref.abs().clamp_min(1.0)[:, None]
    assert float(scaled.max()) <= 1e-6, f"max scaled err {float(scaled.max()):.3g} at v={float(v[scaled.max(1).values.argmax()])}"


@pytest.mark.parametrize(
    "m,n,k", [(8192, 512, 2048), (777, 256, 256), (3, 136, 40), (70000, 128, 512), (4100, 1024, 264)]
)
@pytest.mark.parametrize("variant", [0, 1, 5, 6, 7, 8])
def test_mixed_linear_residual(hip_device, m, n, k, variant):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear_residual

    lin = _linear(k, n, hip_device, 17)
    x32 = _randn((m, k), 19)
    r32 = _randn((m, n), 23, 2.0)
    ref = _ref_linear(x32, lin, False) + r32.double()
    tol = 1e-5 * math.sqrt(k)
    for in_dtype in (torch.float32, torch.float16):
        x = x32.to(hip_device, in_dtype)
        r = r32.to(hip_device)
        y = mixed_linear_residual(x, lin, r, variant=variant)
        assert y.dtype == torch.float32 and y.shape == (m, n)
        _close(y, ref, tol, tol, f"linear+residual in={in_dtype}")
        assert torch.equal(r.cpu(), r32), "residual input modified"
        inplace = mixed_linear_residual(x, lin, r, out=r, variant=variant)
        assert inplace.data_ptr() == r.data_ptr()
        assert torch.equal(inplace.cpu(), y.cpu()), "in-place result differs"


def test_mixed_linear_residual_rejects_bad_inputs(hip_device):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear_residual

    lin = _linear(64, 64, hip_device, 1)
    x = torch.zeros(10, 64, device=hip_device)
    with pytest.raises(ValueError):
        mixed_linear_residual(x, lin, x.half())
    with pytest.raises(ValueError):
        mixed_linear_residual(x, lin, torch.zeros(10, 32, device=hip_device))
    with pytest.raises(ValueError):
        mixed_linear_residual(x, lin, x, out=torch.zeros(10, 64, device=hip_device, dtype=torch.float16))
    with pytest.raises(RuntimeError):
        mixed_linear_residual(x, lin, x, variant=10)


def test_mixed_linear_3d_input(hip_device):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear

    lin = _linear(128, 384, hip_device, 5)
    x = _randn((3, 17, 128), 6)
    y = mixed_linear(x.to(hip_device), lin, output_dtype=torch.float16)
    assert y.shape == (3, 17, 384)
    _close(y.reshape(-1, 384), _ref_linear(x.reshape(-1, 128), lin, False), 2 ** -10, 2 ** -10, "3d")


@pytest.mark.parametrize("d,variant", [(d, v) for d in (32, 64, 128, 256, 512) for v in (1, 2)] + [(256, 3)])
@pytest.mark.parametrize("m", [7, 1000, 8192])
def test_linear_residual_layernorm(hip_device, d, m, variant):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear_add_layer_norm

    lin = _linear(d, d, hip_device, 21)
    norm = _norm(d, hip_device, 22)
    x = _randn((m, d), 23)
    resid = _randn((m, d), 24, 2.0)
    for in_dtype in (torch.float16, torch.float32):
        for out_dtype in (torch.float16, torch.float32):
            r_out, n_out = mixed_linear_add_layer_norm(
                x.to(hip_device, in_dtype), lin, resid.to(hip_device), norm, normalized_dtype=out_dtype,
                variant=variant,
            )
            r64 = _ref_linear(x, lin, False) + resid.double()
            _close(r_out, r64, 2e-5 * math.sqrt(d), 1e-6, "residual_out")
            tol = 5e-5 if out_dtype == torch.float32 else 2 ** -10
            _close(n_out, _ln64(r64, norm), tol, tol, "normalized_out")


@pytest.mark.parametrize("m", [5, 16, 1000, 70001])
def test_linear_layernorm_resident_variant(hip_device, m):
    """Variant 4 (d = K = 256, FP16 X: weights resident in LDS, independent 16-row wave tiles)
    equals variant 1 (the same fragments, MFMA order and epilogue on LDS-staged tiles) bit for
    bit, FP16 and FP32 normalized outputs, ragged row counts and more tiles than waves; FP32 X
    is rejected."""
    from tiktoktechjam2026_amd import _ops

    d = 256
    lin = _linear(d, d, hip_device, 31)
    norm = _norm(d, hip_device, 32)
    x = _randn((m, d), 33).to(hip_device, torch.float16)
    resid = _randn((m, d), 34, 2.0).to(hip_device)
    for out_code in (0, 1):
        r1, n1 = _ops.linear_residual_layer_norm(x, lin.weight, lin.bias, resid, norm.weight, norm.bias,
                                                 float(norm.eps), out_code, 1)
        r4, n4 = _ops.linear_residual_layer_norm(x, lin.weight, lin.bias, resid, norm.weight, norm.bias,
                                                 float(norm.eps), out_code, 4)
        assert torch.equal(r1, r4) and torch.equal(n1, n4), out_code
    r64 = _ref_linear(x.float().cpu(), lin, False) + resid.double().cpu()
    _close(r4, r64, 2e-5 * math.sqrt(d), 1e-6, "resident residual_out")
    _close(n4, _ln64(r64, norm), 2 ** -10, 2 ** -10, "resident normalized_out (FP16)")
    with pytest.raises(RuntimeError):
        _ops.linear_residual_layer_norm(x.float(), lin.weight, lin.bias, resid, norm.weight, norm.bias,
                                        float(norm.eps), 1, 4)


@pytest.mark.parametrize("n,k", [(256, 256), (256, 1024), (256, 136), (512, 512), (512, 2048), (512, 40)])
@pytest.mark.parametrize("m", [7, 300, 5000, 256 * 128 + 77])
def test_linear_residual_layer_norm_wide(hip_device, n, k, m):
    """GEMM tiles holding whole rows with the cross-wave LayerNorm epilogue (n = 256 on
    256 x 256 tiles, n = 512 on 128 x 512 tiles with 32-wide K chunks; any k % 8 == 0):
    ragged rows (m not a multiple of the row tile, and more tiles than workgroups of the
    persistent grid), K not a multiple of the chunk, FP16/FP32 inputs and outputs, and the
    in-place form (residual_out aliasing residual)."""
    from tiktoktechjam2026_amd import _lib
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear_residual_layer_norm

    print(f"\n[wide ln] n={n} k={k} m={m}", flush=True)
    lin = _linear(k, n, hip_device, 25)
    norm = _norm(n, hip_device, 26)
    x = _randn((m, k), 27)
    resid = _randn((m, n), 28, 2.0)
    r64 = _ref_linear(x, lin, False) + resid.double()
    for in_dtype in (torch.float16, torch.float32):
        for out_dtype in (torch.float16, torch.float32):
            r_out, n_out = mixed_linear_residual_layer_norm(
                x.to(hip_device, in_dtype), lin, resid.to(hip_device), norm, normalized_dtype=out_dtype,
            )
            _close(r_out, r64, 2e-5 * math.sqrt(k), 1e-6, "wide residual_out")
            tol = 5e-5 if out_dtype == torch.float32 else 2 ** -10
            _close(n_out, _ln64(r64, norm), tol, tol, "wide normalized_out")
    # in place: residual_out is the residual buffer
    xr = x.to(hip_device, torch.float16)
    rr = resid.to(hip_device).clone()
    nn_out = torch.empty(m, n, device=hip_device, dtype=torch.float16)
    lib = _lib.load()
    _lib.check(
        lib.mpk_linear_add_layernorm(
            xr.data_ptr(), _lib.F16, lin.weight.data_ptr(), lin.bias.data_ptr(), rr.data_ptr(),
            norm.weight.data_ptr(), norm.bias.data_ptr(), rr.data_ptr(), nn_out.data_ptr(), _lib.F16, m, n, k,
            float(norm.eps), _lib.stream_handle(hip_device),
        ),
        "mpk_linear_add_layernorm",
    )
    _close(rr, r64, 2e-5 * math.sqrt(k), 1e-6, "in-place residual_out")
    _close(nn_out, _ln64(r64, norm), 2 ** -10, 2 ** -10, "in-place normalized_out")


def test_linear_residual_layer_norm_wide_rejects(hip_device):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear_residual_layer_norm

    norm = _norm(128, hip_device, 1)
    lin = _linear(256, 128, hip_device, 2)  # out_features not 256 or 512
    with pytest.raises(ValueError):
        mixed_linear_residual_layer_norm(torch.zeros(4, 256, device=hip_device, dtype=torch.float16), lin,
                                         torch.zeros(4, 128, device=hip_device), norm)
    lin2 = _linear(256, 256, hip_device, 3)
    with pytest.raises(ValueError):  # residual on the CPU
        mixed_linear_residual_layer_norm(torch.zeros(4, 256, device=hip_device, dtype=torch.float16), lin2,
                                         torch.zeros(4, 256), _norm(256, hip_device, 4))


@pytest.mark.parametrize("d,f", [(128, 128), (32, 64), (64, 96), (256, 1024), (512, 2048), (128, 512)])
@pytest.mark.parametrize("m", [9, 3000])
@pytest.mark.parametrize("variant", [1, 2])
def test_ffn_residual_layernorm(hip_device, d, f, m, variant):
    _check_ffn(hip_device, d, f, m, variant, torch.float16)


# The wide kernels (d_model 256; variant 3 one wave per SIMD, variant 4 vector + matrix
# waves): one chunk (f 32), no steady chunk (f 64), odd chunk counts, the cfg5 shape; row
# counts below one tile, ragged, and with two or more tiles per workgroup of the persistent
# grid (256 workgroups x 128 rows per pass) and a ragged last tile.
@pytest.mark.parametrize("variant", [3, 4])
@pytest.mark.parametrize("f", [32, 64, 96, 1024])
@pytest.mark.parametrize("m", [9, 3000, 2 * 256 * 128 + 37])
def test_ffn_wide_residual_layernorm(hip_device, f, m, variant):
    _check_ffn(hip_device, 256, f, m, variant, torch.float16)


def test_ffn_wide_fp32_input(hip_device):
    _check_ffn(hip_device, 256, 1024, 777, 4, torch.float32)


def test_ffn_wide_one_wave_rejects_fp32_input(hip_device):
    """Variant 3 (one wave per SIMD) would spill with FP32 X: the library returns
    MPK_EUNSUPPORTED for it before any launch."""
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_ffn_add_layer_norm

    x = torch.zeros(64, 256, device=hip_device)
    with pytest.raises(RuntimeError, match="1002"):
        mixed_ffn_add_layer_norm(
            x, _linear(256, 1024, hip_device, 31), _linear(1024, 256, hip_device, 32), torch.zeros_like(x),
            _norm(256, hip_device, 33), normalized_dtype=torch.float16, variant=3,
        )


def _check_ffn(hip_device, d, f, m, variant, x_dtype):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_ffn_add_layer_norm

    print(f"\n[ffn] d={d} f={f} m={m} variant={variant} x={x_dtype}", flush=True)
    lin_in = _linear(d, f, hip_device, 31)
    lin_out = _linear(f, d, hip_device, 32)
    norm = _norm(d, hip_device, 33)
    x = _randn((m, d), 34)
    resid = _randn((m, d), 35, 2.0)
    for out_dtype in (torch.float16, torch.float32):
        r_out, n_out = mixed_ffn_add_layer_norm(
            x.to(hip_device, x_dtype), lin_in, lin_out, resid.to(hip_device), norm,
            normalized_dtype=out_dtype, variant=variant,
        )
        h = _ref_linear(x, lin_in, True)          # FP32 GELU on the accumulator ...
        h16 = h.float().half()                    # ... rounded to FP16 for the second product
        w = lin_out.weight.detach().cpu().double()
        b = lin_out.bias.detach().cpu().double()
        r64 = h16.double() @ w.t() + b + resid.double()
        # one FP16 ulp of any hidden value may flip against the float64 reference
        atol = 2 ** -11 * float(h.abs().max()) * float(w.abs().max()) * 4 + 2e-5 * math.sqrt(f)
        _close(r_out, r64, atol, 1e-5, "ffn residual_out")
        tol = max(atol * 10, 1e-4) if out_dtype == torch.float32 else 2 ** -9
        _close(n_out, _ln64(r64, norm), tol, tol, "ffn normalized_out")
        # a last layer: N' written into a given tensor, or returned alone, with R' not stored
        # (residual_out NULL at the C ABI) - the same N' bit for bit
        buf = torch.full_like(n_out, float("nan"))
        r_none, n_into = mixed_ffn_add_layer_norm(
            x.to(hip_device, x_dtype), lin_in, lin_out, resid.to(hip_device), norm,
            normalized_dtype=out_dtype, variant=variant, out=buf, store_residual=False,
        )
        assert r_none is None and n_into.data_ptr() == buf.data_ptr() and torch.equal(buf, n_out)
        r_none, n_final = mixed_ffn_add_layer_norm(
            x.to(hip_device, x_dtype), lin_in, lin_out, resid.to(hip_device), norm,
            normalized_dtype=out_dtype, variant=variant, store_residual=False,
        )
        assert r_none is None and torch.equal(n_final, n_out)


def test_fused_ops_reject_unsupported(hip_device):
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_ffn_add_layer_norm, mixed_linear_add_layer_norm

    lin = _linear(96, 96, hip_device, 1)
    norm = _norm(96, hip_device, 1)
    x = torch.zeros(4, 96, device=hip_device, dtype=torch.float16)
    r = torch.zeros(4, 96, device=hip_device)
    with pytest.raises(ValueError):
        mixed_linear_add_layer_norm(x, lin, r, norm)
    with pytest.raises(ValueError):
        mixed_ffn_add_layer_norm(x, lin, lin, r, norm)


# --------------------------------------------------------------------------- attention


def _ref_attention(q, k, v, scale, causal, key_valid=None):
    q = q.detach().cpu().half().double()
    k = k.detach().cpu().half().double()
    v = v.detach().cpu().half().double()
    s = (q @ k.transpose(-1, -2)) * scale
    S = q.shape[-2]
    if causal:
        s = s.masked_fill(torch.ones(S, S, dtype=torch.bool).triu(1), float("-inf"))
    if key_valid is not None:
        s = s.masked_fill(~key_valid.cpu()[:, None, None, :], float("-inf"))
    p = torch.softmax(s, dim=-1)
    return (p @ v).permute(0, 2, 1, 3)  # [B, S, H, hd]


def _packed_qkv(b, s, h, hd, seed, device, dtype):
    qkv = _randn((b, s, 3, h, hd), seed, 1.5).to(device, dtype)
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    return qkv, q, k, v


@pytest.mark.parametrize(
    "b,h,s,hd",
    [(2, 4, 128, 32), (2, 2, 256, 16), (1, 8, 300, 64), (1, 2, 77, 128), (3, 4, 1024, 32), (1, 1, 1, 32),
     (2, 3, 65, 16), (1, 2, 2048, 64), (2, 16, 128, 8), (1, 4, 333, 8), (2, 4, 128, 256), (1, 2, 517, 256)],
)
@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5])
def test_fp16_causal_attention(hip_device, b, h, s, hd, variant):
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention, fp16_causal_attention, is_fp16_supported

    _, q, k, v = _packed_qkv(b, s, h, hd, 41, hip_device, torch.float16)
    scale = hd ** -0.5
    assert is_fp16_supported(q, k, v, True)
    out = attention(q, k, v, scale, causal=True, variant=variant)
    assert out.shape == (b, s, h, hd) and out.dtype == torch.float16 and out.is_contiguous()
    ref = _ref_attention(q, k, v, scale, True)
    # P is rounded to FP16 for the P.V product and the output is stored as FP16
    _close(out, ref, 3e-3, 3e-3, "fp16 causal attention")
    if variant == 1:
        _close(fp16_causal_attention(q, k, v, scale), ref, 3e-3, 3e-3, "fp16_causal_attention")


@pytest.mark.parametrize(
    "b,h,s,hd",
    [(2, 4, 128, 32), (1, 8, 300, 64), (3, 4, 1024, 32), (1, 1, 1, 32), (2, 3, 65, 64), (1, 2, 2048, 64),
     (1, 2, 4096, 32), (2, 2, 33, 32), (1, 3, 517, 64)],
)
@pytest.mark.parametrize("variant", [6, 7, 8])
def test_fp16_causal_attention_32x32(hip_device, b, h, s, hd, variant):
    """The 32x32-MFMA kernel (head_dim 32 / 64) against the float64 reference."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention

    _, q, k, v = _packed_qkv(b, s, h, hd, 47, hip_device, torch.float16)
    scale = hd ** -0.5
    out = attention(q, k, v, scale, causal=True, variant=variant)
    assert out.shape == (b, s, h, hd) and out.dtype == torch.float16 and out.is_contiguous()
    _close(out, _ref_attention(q, k, v, scale, True), 3e-3, 3e-3, "fp16 causal attention (32x32)")


@pytest.mark.parametrize("variant", [6, 7, 8])
def test_attention_32x32_noncausal_fp32io_keymask_negative_scale(hip_device, variant):
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention

    for b, h, s, hd in ((2, 4, 130, 32), (1, 2, 200, 64)):
        _, q, k, v = _packed_qkv(b, s, h, hd, 53, hip_device, torch.float32)
        scale = hd ** -0.5
        out = attention(q, k, v, scale, causal=False, variant=variant)
        assert out.dtype == torch.float32
        _close(out, _ref_attention(q, k, v, scale, False), 3e-3, 3e-3, "non-causal fp32 io (32x32)")
        out_h = attention(q.half(), k.half(), v.half(), scale, causal=False, variant=variant)
        _close(out_h, _ref_attention(q, k, v, scale, False), 3e-3, 3e-3, "non-causal fp16 io (32x32)")
        out_n = attention(q.half(), k.half(), v.half(), -scale, causal=True, variant=variant)
        _close(out_n, _ref_attention(q, k, v, -scale, True), 3e-3, 3e-3, "negative scale (32x32)")
        lengths = torch.tensor([max(1, s - 37 * (i + 1)) for i in range(b)])
        key_valid = (torch.arange(s)[None, :] < lengths[:, None]).to(hip_device)
        key_valid[:, 0] = False  # the first key masked: rows see their first valid key in a later tile
        out_m = attention(q.half(), k.half(), v.half(), scale, causal=True, key_valid=key_valid, variant=variant)
        ref_m = _ref_attention(q, k, v, scale, True, key_valid)
        rows_with_keys = torch.isfinite(ref_m).all(dim=-1)
        _close(out_m.cpu()[rows_with_keys], ref_m[rows_with_keys], 3e-3, 3e-3, "key mask (32x32)")


@pytest.mark.parametrize("variant", [1, 6, 7, 8])
@pytest.mark.parametrize("pattern", ["ramp", "spikes"])
def test_attention_rising_scores(hip_device, variant, pattern):
    """Scores that keep rising along the sequence: the running max has to be raised
    in tiles after the first (for the 32x32 kernel, through its exact-max fallback),
    including weights that would overflow FP16 against a stale max."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention

    for b, h, s, hd in ((2, 2, 1024, 32), (1, 2, 600, 64)):
        qkv = _randn((b, s, 3, h, hd), 61, 1.0)
        if pattern == "ramp":  # key norms grow 40x over the sequence
            qkv[:, :, 1] *= torch.linspace(0.25, 10.0, s)[None, :, None, None]
        else:  # a few keys far larger than everything before them
            for pos, mult in ((130, 6.0), (400, 12.0), (s - 50, 20.0)):
                qkv[:, pos, 1] *= mult
        qkv = qkv.to(hip_device, torch.float16)
        q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
        scale = hd ** -0.5
        out = attention(q, k, v, scale, causal=True, variant=variant)
        assert torch.isfinite(out).all()
        _close(out, _ref_attention(q, k, v, scale, True), 3e-3, 3e-3, f"rising scores ({pattern})")


@pytest.mark.parametrize("variant", [6, 7, 8])
@pytest.mark.parametrize("pattern", ["ramp", "spikes"])
def test_attention_prescaled_rising_scores(hip_device, variant, pattern):
    """Pre-scaled q with scores that keep rising: steady head-dim-32 tiles (accumulators started
    at -m) raise the row max through their exact-max fallback, head dim 64 and 128-key tiles
    through the ordinary score test with c = 1; weights that would overflow FP16 against a stale
    max included."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention_prescaled

    for b, h, s, hd in ((2, 2, 1024, 32), (1, 2, 600, 64), (1, 2, 2048, 64)):
        qkv = _randn((b, s, 3, h, hd), 61, 1.0)
        if pattern == "ramp":
            qkv[:, :, 1] *= torch.linspace(0.25, 10.0, s)[None, :, None, None]
        else:
            for pos, mult in ((130, 6.0), (400, 12.0), (s - 50, 20.0)):
                qkv[:, pos, 1] *= mult
        scale = hd ** -0.5
        c = float(torch.tensor(scale, dtype=torch.float32) * torch.tensor(1.4426950408889634, dtype=torch.float32))
        qkv_ps = qkv.clone()
        qkv_ps[:, :, 0] *= c
        qkv16 = qkv.to(hip_device, torch.float16)
        q, k, v = qkv16.permute(2, 0, 3, 1, 4).unbind(0)
        qs = qkv_ps.to(hip_device, torch.float16).permute(2, 0, 3, 1, 4)[0]
        out = attention_prescaled(qs, k, v, causal=True, variant=variant)
        assert torch.isfinite(out).all()
        # the reference takes the kernel's own FP16 q * c, so large scores do not magnify the
        # difference between rounding q and rounding q * c: softmax(q' k^T ln 2) = 2^(q' k^T)
        ref = _ref_attention(qs, k, v, 1.0 / 1.4426950408889634, True)
        _close(out, ref, 3e-3, 3e-3, f"pre-scaled rising scores ({pattern}, hd {hd})")


@pytest.mark.parametrize("variant", [6, 7])
def test_attention_prescaled_wide_row_max(hip_device, variant):
    """Pre-scaled q whose row maxima grow past the range in which the kernel keeps them as FP16
    values (|m| >= 2048 in log2 units): keys of the second half 60x larger, so each wave
    switches from the MFMA-initialised steady tiles to the FP32 splat mid-row; batch row 1
    keeps ordinary scores.  Against float64 of the kernel's own q."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention_prescaled

    b, h, s, hd = 2, 2, 1024, 32
    qkv = _randn((b, s, 3, h, hd), 71, 1.0)
    qkv[0, s // 2:, 1] *= 60.0
    qkv[0, :, 0] *= 15.0
    qkv16 = qkv.to(hip_device, torch.float16)
    q, k, v = qkv16.permute(2, 0, 3, 1, 4).unbind(0)
    c = float(torch.tensor(hd ** -0.5, dtype=torch.float32) * torch.tensor(1.4426950408889634, dtype=torch.float32))
    qs = (q.float() * c).half()
    out = attention_prescaled(qs, k, v, causal=True, variant=variant)
    assert torch.isfinite(out).all()
    ref = _ref_attention(qs, k, v, 1.0 / 1.4426950408889634, True)
    top = (qs[0].double().cpu() @ k[0].double().cpu().transpose(-1, -2)).amax()
    assert float(top) > 4096, float(top)  # the test reaches the wide range
    _close(out, ref, 3e-3, 3e-3, "pre-scaled attention, row maxima past 2048")


@pytest.mark.parametrize("variant", [6, 7])
def test_attention_32x32_grouped_schedule(hip_device, variant):
    """A launch with at least 1024 workgroups per XCD walks its (batch, head) rows in groups
    of 8 (B 64 x H 8 = 512 rows; S 2048 gives 16 query blocks of 128 for variant 6, S 4096
    16 blocks of 256 for variant 7).  Batch rows are independent and a block's arithmetic
    does not depend on when it runs, so the grouped launch must equal, bit for bit, eight
    launches of 8 sequences each (64 rows: too few workgroups for grouping); two rows are
    also checked against float64."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention

    b, h, hd = 64, 8, 32
    s = 2048 if variant == 6 else 4096
    print(f"\n[attention grouped] b={b} h={h} s={s} variant={variant}", flush=True)
    torch.manual_seed(5)
    qkv = (torch.randn(b, s, 3, h, hd) * 1.5).to(hip_device, torch.float16)
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    grouped = attention(q, k, v, hd ** -0.5, causal=True, variant=variant)
    for b0 in range(0, b, 8):
        part = attention(q[b0:b0 + 8], k[b0:b0 + 8], v[b0:b0 + 8], hd ** -0.5, causal=True, variant=variant)
        assert torch.equal(grouped[b0:b0 + 8], part), f"sequences {b0}..{b0 + 7} differ"
    for row in (9, 500):
        bi, hi = divmod(row, h)
        ref = _ref_attention(q[bi:bi + 1, hi:hi + 1], k[bi:bi + 1, hi:hi + 1], v[bi:bi + 1, hi:hi + 1], hd ** -0.5, True)
        _close(grouped[bi:bi + 1, :, hi:hi + 1], ref, 3e-3, 3e-3, f"grouped attention row {row}")


def test_attention_32x32_rejects_other_head_dims(hip_device):
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention

    _, q, k, v = _packed_qkv(1, 64, 2, 16, 59, hip_device, torch.float16)
    with pytest.raises(RuntimeError):
        attention(q, k, v, 0.25, causal=True, variant=6)


@pytest.mark.parametrize("b,h,s,hd", [(2, 4, 128, 32), (1, 2, 200, 64), (2, 2, 96, 16), (2, 4, 70, 8), (1, 2, 90, 256)])
def test_attention_noncausal_fp32io_and_keymask(hip_device, b, h, s, hd):
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention, causal_attention

    _, q, k, v = _packed_qkv(b, s, h, hd, 43, hip_device, torch.float32)
    scale = hd ** -0.5
    out = attention(q, k, v, scale, causal=False)
    assert out.dtype == torch.float32
    _close(out, _ref_attention(q, k, v, scale, False), 3e-3, 3e-3, "non-causal fp32 io")
    _close(causal_attention(q, k, v, scale), _ref_attention(q, k, v, scale, True), 3e-3, 3e-3, "causal fp32 io")
    lengths = torch.tensor([max(1, s - 17 * (i + 1)) for i in range(b)])
    key_valid = (torch.arange(s)[None, :] < lengths[:, None]).to(hip_device)
    out_m = attention(q.half(), k.half(), v.half(), scale, causal=True, key_valid=key_valid)
    ref_m = _ref_attention(q, k, v, scale, True, key_valid)
    _close(out_m, ref_m, 3e-3, 3e-3, "causal + key mask")


@pytest.mark.parametrize(
    "hd,variant", [(32, 1), (32, 6), (32, 7), (64, 6), (64, 2), (16, 1), (8, 1), (128, 1), (256, 1)]
)
@pytest.mark.parametrize("mags", [(1e5, 1e-5, 1e5), (1e-6, 1e6, 1e-6), (1e5, 1e-5, 1e-6)])
def test_attention_fp32io_exponent_range(hip_device, hd, variant, mags):
    """FP32 inputs far outside FP16's normal range (about 6e-5 .. 65504), as the reference's
    TF32 kernel accepts them: |q| up to ~5e5 with |k| ~ 1e-5 (scores stay O(1), so the
    softmax is not degenerate), the mirror image, and v below FP16's normal range.  The
    kernels scale q, k and v by powers of two before rounding them to FP16, so nothing
    overflows or loses precision to subnormals; compared with float64 on the unrounded
    FP32 values, relative to the size of v."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention

    b, h, s = 2, 2, 300
    sq, sk, sv = mags
    print(f"\n[attention fp32 range] hd={hd} variant={variant} q~{sq:g} k~{sk:g} v~{sv:g}", flush=True)
    g = torch.Generator().manual_seed(61)
    qkv = torch.randn(b, s, 3, h, hd, generator=g)
    qkv[:, :, 0] *= sq
    qkv[:, :, 1] *= sk
    qkv[:, :, 2] *= sv
    qkv = qkv.to(hip_device)
    q, k, v = qkv.permute(2, 0, 3, 1, 4).unbind(0)
    scale = hd ** -0.5
    for causal in (True, False):
        out = attention(q, k, v, scale, causal=causal, variant=variant)
        assert out.dtype == torch.float32 and torch.isfinite(out).all()
        q64, k64, v64 = (t.detach().cpu().double() for t in (q, k, v))
        sc = (q64 @ k64.transpose(-1, -2)) * scale
        if causal:
            sc = sc.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
        ref = (torch.softmax(sc, dim=-1) @ v64).permute(0, 2, 1, 3)
        err = (out.cpu().double() - ref).abs().max().item()
        assert err <= 3e-3 * sv, f"max error {err:g} against |v| ~ {sv:g} (causal={causal})"


def test_attention_causality_exact(hip_device):
    """Output row t is bit-identical when keys/values after t change."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention

    qkv, q, k, v = _packed_qkv(2, 512, 4, 32, 45, hip_device, torch.float16)
    base = attention(q, k, v, 32 ** -0.5)
    t = 300
    qkv2 = qkv.clone()
    qkv2[:, t + 1:] = _randn(tuple(qkv2[:, t + 1:].shape), 46).to(hip_device, torch.float16)
    q2, k2, v2 = qkv2.permute(2, 0, 3, 1, 4).unbind(0)
    moved = attention(q2, k2, v2, 32 ** -0.5)
    assert torch.equal(base[:, : t + 1], moved[:, : t + 1])
    assert not torch.equal(base[:, t + 1:], moved[:, t + 1:])


def test_attention_rejects_unsupported(hip_device):
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention, is_fp16_supported

    x = torch.zeros(1, 2, 16, 24, device=hip_device, dtype=torch.float16)
    assert not is_fp16_supported(x, x, x, True)
    with pytest.raises(ValueError):
        attention(x, x, x, 1.0)


# --------------------------------------------------------------------------- whole-layer fusions


def _ln_module_ref(r64, norm):
    return _ln64(r64, norm)


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("m", [5, 1000, 9000])
@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_layer_norm_qkv(hip_device, d, m, variant):
    from tiktoktechjam2026_amd.mixed_precision.hip_fused import layer_norm_qkv

    x = _randn((m, d), 51, 2.0)
    norm = _norm(d, hip_device, 52)
    lin = _linear(d, 3 * d, hip_device, 53)
    qkv = layer_norm_qkv(x.to(hip_device), norm, lin, variant=variant)
    assert qkv.dtype == torch.float16 and qkv.shape == (m, 3 * d)
    n16 = _ln64(x.double(), norm).float().half()
    ref = n16.double() @ lin.weight.detach().cpu().double().t() + lin.bias.detach().cpu().double()
    # an FP16 rounding flip of a normalized value moves an output by <= ulp * |w|
    _close(qkv, ref, 2 ** -9, 2 ** -10, "layer_norm_qkv")


@pytest.mark.parametrize("d,f", [(128, 128), (32, 64), (64, 256), (32, 32)])
@pytest.mark.parametrize("m", [7, 4100])
@pytest.mark.parametrize("last", [False, True])
@pytest.mark.parametrize("variant", [0, 1, 2, 3])
def test_fused_layer_tail(hip_device, d, f, m, last, variant):
    _check_layer_tail(hip_device, d, f, m, last, variant)


# Row counts that give every workgroup of the persistent grid at least two tiles, with a
# ragged last tile on the second pass (d 32/64: 512 workgroups x 128 rows; d 128: 256 x 128;
# variant 3 has 64-row tiles, so the same counts give it four or more passes).
@pytest.mark.parametrize("d,f,m", [(32, 64, 2 * 512 * 128 + 37), (64, 256, 2 * 512 * 128 + 37),
                                   (128, 128, 2 * 256 * 128 + 37)])
@pytest.mark.parametrize("last", [False, True])
@pytest.mark.parametrize("variant", [1, 2, 3])
def test_fused_layer_tail_multi_pass(hip_device, d, f, m, last, variant):
    _check_layer_tail(hip_device, d, f, m, last, variant)


def _check_layer_tail(hip_device, d, f, m, last, variant):
    from tiktoktechjam2026_amd.mixed_precision.hip_fused import fused_layer_tail

    ctx = _randn((m, d), 61)
    x = _randn((m, d), 62, 2.0)
    out_proj = _linear(d, d, hip_device, 63)
    ffn_in = _linear(d, f, hip_device, 64)
    ffn_out = _linear(f, d, hip_device, 65)
    norm2 = _norm(d, hip_device, 66)
    next_norm = _norm(d, hip_device, 67)
    qkv_proj = None if last else _linear(d, 3 * d, hip_device, 68)
    x_out, out = fused_layer_tail(
        ctx.to(hip_device, torch.float16), x.to(hip_device), out_proj, norm2, ffn_in, ffn_out, next_norm, qkv_proj,
        variant=variant,
    )
    W = lambda lin: lin.weight.detach().cpu().double()  # noqa: E731
    B = lambda lin: lin.bias.detach().cpu().double()  # noqa: E731
    x1 = ctx.half().double() @ W(out_proj).t() + B(out_proj) + x.double()
    n2 = _ln64(x1, norm2).float().half().double()
    h = n2 @ W(ffn_in).t() + B(ffn_in)
    h = (0.5 * h * (1.0 + torch.erf(h / math.sqrt(2.0)))).float().half().double()
    x2 = h @ W(ffn_out).t() + B(ffn_out) + x1
    # FP16 rounding flips of n2 / h against the float64 chain bound the residual error
    _close(x_out, x2, 3e-3, 1e-4, "layer tail residual")
    n1 = _ln64(x2, next_norm)
    if last:
        assert out.dtype == torch.float32 and out.shape == (m, d)
        _close(out, n1, 5e-3, 5e-3, "layer tail final norm")
    else:
        assert out.dtype == torch.float16 and out.shape == (m, 3 * d)
        ref = n1.float().half().double() @ W(qkv_proj).t() + B(qkv_proj)
        _close(out, ref, 5e-3, 5e-3, "layer tail qkv")



def _check_q_scaled(scaled, plain, d, c, what):
    """q columns [0, d) of a q-scaled QKV against the unscaled launch's times c: both are one FP16
    rounding of the same FP32 value (times c), so they differ by at most about one FP16 ulp of
    the result; k / v columns bit for bit."""
    assert scaled.dtype == plain.dtype == torch.float16 and scaled.shape == plain.shape
    assert torch.equal(scaled[..., d:], plain[..., d:]), what
    q_s = scaled[..., :d].cpu().double()
    q_u = plain[..., :d].cpu().double() * c
    err = (q_s - q_u).abs()
    bound = 2.0 ** -10 * q_u.abs() + 2.0 ** -24  # one ulp at the result's binade, FP16 subnormals
    assert bool((err <= bound).all()), f"{what}: max err {float(err.max()):.3g}"
    assert not torch.equal(scaled[..., :d], plain[..., :d]), f"{what}: q left unscaled"


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("m", [5, 9000])
@pytest.mark.parametrize("variant", [0, 1, 3])
def test_layer_norm_qkv_q_scaled(hip_device, d, m, variant):
    """mpk_layernorm_qkv_qscaled: the q columns scaled in FP32 before the FP16 rounding, k / v
    columns those of mpk_layernorm_qkv bit for bit."""
    from tiktoktechjam2026_amd.mixed_precision.hip_fused import layer_norm_qkv

    x = _randn((m, d), 51, 2.0).to(hip_device)
    norm = _norm(d, hip_device, 52)
    lin = _linear(d, 3 * d, hip_device, 53)
    c = 0.25503486
    plain = layer_norm_qkv(x, norm, lin, variant=variant)
    scaled = layer_norm_qkv(x, norm, lin, variant=variant, q_scale=c)
    _check_q_scaled(scaled, plain, d, c, "layer_norm_qkv q_scale")


@pytest.mark.parametrize("d,f", [(128, 128), (32, 64), (64, 256)])
@pytest.mark.parametrize("m", [7, 2 * 256 * 128 + 37])
@pytest.mark.parametrize("variant", [0, 1, 3])
def test_fused_layer_tail_q_scaled(hip_device, d, f, m, variant):
    """mpk_layer_tail_qscaled: residual output and k / v columns of the next QKV equal
    mpk_layer_tail's bit for bit, the q columns are scaled before the FP16 rounding; the last
    layer ignores the factor."""
    from tiktoktechjam2026_amd.mixed_precision.hip_fused import fused_layer_tail

    ctx = _randn((m, d), 61).to(hip_device, torch.float16)
    x = _randn((m, d), 62, 2.0).to(hip_device)
    mods = [_linear(d, d, hip_device, 63), _norm(d, hip_device, 66), _linear(d, f, hip_device, 64),
            _linear(f, d, hip_device, 65), _norm(d, hip_device, 67)]
    qkv_proj = _linear(d, 3 * d, hip_device, 68)
    c = 0.17677669 * 1.4426950
    x_p, qkv_p = fused_layer_tail(ctx, x, *mods, qkv_proj, variant=variant)
    x_s, qkv_s = fused_layer_tail(ctx, x, *mods, qkv_proj, variant=variant, q_scale=c)
    assert torch.equal(x_p, x_s)
    _check_q_scaled(qkv_s, qkv_p, d, c, "layer tail q_scale")
    x_l, n_l = fused_layer_tail(ctx, x, *mods, None, variant=variant)
    x_ls, n_ls = fused_layer_tail(ctx, x, *mods, None, variant=variant, q_scale=c)
    assert torch.equal(x_l, x_ls) and torch.equal(n_l, n_ls)


def test_q_scale_rejects(hip_device):
    from tiktoktechjam2026_amd.mixed_precision.hip_fused import layer_norm_qkv

    x = _randn((4, 32), 51).to(hip_device)
    with pytest.raises(ValueError):
        layer_norm_qkv(x, _norm(32, hip_device, 52), _linear(32, 96, hip_device, 53), q_scale=float("nan"))
    with pytest.raises(ValueError):
        layer_norm_qkv(x, _norm(32, hip_device, 52), _linear(32, 96, hip_device, 53), q_scale=0.0)


# --------------------------------------------------------------------------- attention inside the layer tail


@pytest.mark.parametrize("d,f,heads", [(128, 128, 4), (64, 256, 2), (64, 64, 2), (32, 32, 1), (32, 128, 1),
                                         (32, 64, 2), (64, 128, 4), (32, 32, 2)])
@pytest.mark.parametrize("b,s", [(1, 64), (3, 128), (2, 256)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("last", [False, True])
def test_attention_layer_tail_matches_two_kernels(hip_device, d, f, heads, b, s, causal, last):
    """mpk_attention_layer_tail (head dim 32 or 16) equals mpk_causal_attention (variant 1: the
    16x16 kernel, 64-key tiles) followed by mpk_layer_tail (variant 3: 4 waves x 16 rows), bit for bit:
    the attention stage runs the same arithmetic over the same tiles, and the tail is the
    same kernel.  The two-kernel result is itself checked against float64 by the tests
    above."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention
    from tiktoktechjam2026_amd.mixed_precision.hip_fused import fused_attention_layer_tail, fused_layer_tail

    hd = d // heads
    print(f"\n[attention tail] d={d} f={f} heads={heads} b={b} s={s} causal={causal} last={last}", flush=True)
    qkv = (_randn((b, s, 3 * d), 71, 1.5)).to(hip_device, torch.float16)
    x = _randn((b, s, d), 72, 2.0).to(hip_device)
    out_proj = _linear(d, d, hip_device, 73)
    ffn_in = _linear(d, f, hip_device, 74)
    ffn_out = _linear(f, d, hip_device, 75)
    norm2 = _norm(d, hip_device, 76)
    next_norm = _norm(d, hip_device, 77)
    qkv_proj = None if last else _linear(d, 3 * d, hip_device, 78)
    scale = hd ** -0.5
    x_f, out_f = fused_attention_layer_tail(qkv, x, heads, scale, causal, out_proj, norm2, ffn_in, ffn_out,
                                            next_norm, qkv_proj)
    q, k, v = qkv.view(b, s, 3, heads, hd).permute(2, 0, 3, 1, 4).unbind(0)
    ctx = attention(q, k, v, scale, causal=causal, variant=1).reshape(b, s, d)
    x_u, out_u = fused_layer_tail(ctx, x, out_proj, norm2, ffn_in, ffn_out, next_norm, qkv_proj, variant=3)
    assert torch.equal(x_f, x_u), (x_f - x_u).abs().max().item()
    assert out_f.dtype == out_u.dtype and torch.equal(out_f, out_u), (out_f.float() - out_u.float()).abs().max().item()


def test_attention_layer_tail_rejects(hip_device):
    """Ragged sequences (not whole 64-row tiles), other head dims and an output that overlaps
    the input QKV are refused before any launch."""
    from tiktoktechjam2026_amd import _lib
    from tiktoktechjam2026_amd.mixed_precision.hip_fused import fused_attention_layer_tail

    d, f = 128, 128
    mods = [_linear(d, d, hip_device, 1), _norm(d, hip_device, 2), _linear(d, f, hip_device, 3),
            _linear(f, d, hip_device, 4), _norm(d, hip_device, 5), _linear(d, 3 * d, hip_device, 6)]
    for s, heads in ((96, 4), (128, 2), (128, 8)):  # ragged; head dim 64; head dim 16 at d_model 128
        qkv = torch.zeros(1, s, 3 * d, device=hip_device, dtype=torch.float16)
        x = torch.zeros(1, s, d, device=hip_device)
        with pytest.raises(ValueError):
            fused_attention_layer_tail(qkv, x, heads, 0.1, True, *mods)
    # at the C ABI: the next layer's QKV written over this layer's
    m = 128
    qkv = torch.zeros(m, 3 * d, device=hip_device, dtype=torch.float16)
    x = torch.zeros(m, d, device=hip_device)
    x_out = torch.empty_like(x)
    out_proj, norm2, ffn_in, ffn_out, next_norm, qkv_proj = mods
    lib = _lib.load()
    status = lib.mpk_attention_layer_tail(
        qkv.data_ptr(), x.data_ptr(), out_proj.weight.data_ptr(), out_proj.bias.data_ptr(), norm2.weight.data_ptr(),
        norm2.bias.data_ptr(), ffn_in.weight.data_ptr(), ffn_in.bias.data_ptr(), ffn_out.weight.data_ptr(),
        ffn_out.bias.data_ptr(), next_norm.weight.data_ptr(), next_norm.bias.data_ptr(), qkv_proj.weight.data_ptr(),
        qkv_proj.bias.data_ptr(), x_out.data_ptr(), qkv.data_ptr(), 0, m, d, f, 4, 128, 0.1, 1, 1e-5, 1e-5,
        _lib.stream_handle(qkv.device),
    )
    assert status == _lib.MPK_EINVAL


# --------------------------------------------------------------------------- pre-scaled q


@pytest.mark.parametrize("m,n,k,q_cols", [(130, 768, 256, 256), (8192, 384, 128, 128), (257, 40, 24, 16), (64, 96, 32, 0)])
@pytest.mark.parametrize("variant", [0, 1, 5, 7, 8, 9])
def test_linear_q_scaled(hip_device, m, n, k, q_cols, variant):
    """The QKV projection with the attention scale folded into q: columns from q_cols on equal
    mpk_linear's bit for bit (the same kernel, times 1), the first q_cols are (x W^T + b) * c
    rounded to FP16 once."""
    from tiktoktechjam2026_amd.mixed_precision.hip_linear import mixed_linear, mixed_linear_q_scaled

    x = _randn((m, k), 91, 1.0).to(hip_device, torch.float16)
    lin = _linear(k, n, hip_device, 92)
    c = 0.25503486
    y = mixed_linear_q_scaled(x, lin, q_cols, c, variant=variant)
    plain = mixed_linear(x, lin, output_dtype=torch.float16, variant=variant)
    assert y.dtype == torch.float16 and y.shape == (m, n)
    assert torch.equal(y[:, q_cols:], plain[:, q_cols:])
    if q_cols:
        ref = _ref_linear(x, lin, False)[:, :q_cols] * c
        err = (y[:, :q_cols].cpu().double() - ref).abs()
        assert float((err / ref.abs().clamp_min(1e-3)).max()) < 2e-3, float(err.max())


@pytest.mark.parametrize(
    "b,h,s,hd", [(2, 4, 256, 32), (1, 8, 300, 64), (3, 4, 1024, 32), (1, 2, 4096, 32), (2, 2, 33, 32), (1, 3, 517, 64)]
)
@pytest.mark.parametrize("variant", [0, 6, 7, 8])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_prescaled(hip_device, b, h, s, hd, variant, causal):
    """attention_prescaled over q * scale * log2(e) (rounded to FP16 once) against the float64
    reference of the unscaled problem, with and without a key mask."""
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention_prescaled

    qkv = _randn((b, s, 3, h, hd), 97, 1.5)
    scale = hd ** -0.5
    c = float(torch.tensor(scale, dtype=torch.float32) * torch.tensor(1.4426950408889634, dtype=torch.float32))
    qkv_ps = qkv.clone()
    qkv_ps[:, :, 0] *= c
    qkv16, qkv_ps16 = qkv.to(hip_device, torch.float16), qkv_ps.to(hip_device, torch.float16)
    q, k, v = qkv16.permute(2, 0, 3, 1, 4).unbind(0)
    qs = qkv_ps16.permute(2, 0, 3, 1, 4)[0]
    out = attention_prescaled(qs, k, v, causal=causal, variant=variant)
    assert out.shape == (b, s, h, hd) and out.dtype == torch.float16 and out.is_contiguous()
    # the reference takes the unscaled q in FP32 (its FP16 rounding differs from that of q c)
    ref = _ref_attention(qkv[:, :, 0].permute(0, 2, 1, 3).float(), k, v, scale, causal)
    _close(out, ref, 4e-3, 4e-3, "pre-scaled attention")
    lengths = torch.tensor([max(1, s - 29 * (i + 1)) for i in range(b)])
    key_valid = (torch.arange(s)[None, :] < lengths[:, None]).to(hip_device)
    out_m = attention_prescaled(qs, k, v, causal=causal, key_valid=key_valid, variant=variant)
    ref_m = _ref_attention(qkv[:, :, 0].permute(0, 2, 1, 3).float(), k, v, scale, causal, key_valid)
    rows = torch.isfinite(ref_m).all(dim=-1)
    _close(out_m.cpu()[rows], ref_m[rows], 4e-3, 4e-3, "pre-scaled attention, key mask")


def test_attention_prescaled_rejects(hip_device):
    from tiktoktechjam2026_amd.custom_kernel.hip_attention import attention_prescaled

    _, q, k, v = _packed_qkv(1, 64, 2, 16, 5, hip_device, torch.float16)
    with pytest.raises(ValueError):
        attention_prescaled(q, k, v)  # head dim 16: the 16x16 kernel has no pre-scaled form
    _, q, k, v = _packed_qkv(1, 64, 2, 32, 5, hip_device, torch.float16)
    with pytest.raises(ValueError):
        attention_prescaled(q, k, v, variant=1)
    _, q, k, v = _packed_qkv(1, 64, 2, 32, 5, hip_device, torch.float32)
    with pytest.raises(ValueError):
        attention_prescaled(q, k, v)
