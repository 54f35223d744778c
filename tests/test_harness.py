"""Harness semantics pinned on hand-built tensors (CPU): the accuracy rule of
``torch_transformer_benchmark.py:503-570``, percentiles, microbatch wrappers."""

from __future__ import annotations

import math

import pytest
import torch

from tiktoktechjam2026_amd import harness
from tiktoktechjam2026_amd.config import TransformerConfig


def test_rule_abs_or_rel_branch():
    ref = torch.tensor([0.0, 1.0, 100.0, -2.0, 0.5])
    #                    abs ok   abs ok  rel ok (1.9)  rel fail     abs fail/rel ok?
    opt = torch.tensor([0.002, 0.998, 101.9, -2.05, 0.5 + 0.009])
    result = harness.compare_outputs(ref, opt, rtol=0.02, atol=0.002)
    # -2.05: |d| = 0.05 > 0.002 and > 0.04 -> fails; 0.509: |d| = 0.009 <= 0.01 -> passes (rel)
    assert result.failed_elements == 1
    assert result.failed_feature_dims == [3]
    assert result.worst_index == (2,)
    assert math.isclose(result.max_abs_error, 1.9, rel_tol=1e-6)


def test_rule_is_not_isclose():
    # torch.isclose uses atol + rtol*|ref| (more permissive); the rule is an OR of the two bounds
    ref = torch.tensor([0.05])
    opt = torch.tensor([0.05 + 0.0025])  # 0.0025 > 0.002 and > 0.001, but <= 0.002 + 0.001
    assert torch.isclose(opt, ref, rtol=0.02, atol=0.002).all()
    assert harness.compare_outputs(ref, opt, rtol=0.02, atol=0.002).failed_elements == 1


def test_rule_exact_boundary_and_zero_reference():
    ref = torch.tensor([0.0, 0.0])
    opt = torch.tensor([0.001953125, 0.00201])  # exactly representable 2^-9 passes; 0.00201 fails
    result = harness.compare_outputs(ref, opt, rtol=0.02, atol=0.001953125)
    assert result.failed_elements == 1
    # relative error with a zero reference uses the 1e-12 clamp
    assert result.max_relative_error > 1e9


def test_rule_non_finite_fails():
    ref = torch.tensor([1.0, float("nan"), 1.0, float("inf")])
    opt = torch.tensor([float("nan"), 1.0, float("inf"), float("inf")])
    result = harness.compare_outputs(ref, opt, rtol=0.02, atol=0.002)
    assert result.failed_elements == 4
    assert not result.passed


def test_shape_mismatch_raises():
    with pytest.raises(AssertionError):
        harness.compare_outputs(torch.zeros(2, 3), torch.zeros(3, 2), 0.02, 0.002)


def test_failed_feature_dims_reduce_over_leading_dims():
    ref = torch.zeros(2, 3, 4)
    opt = ref.clone()
    opt[1, 2, 3] = 1.0
    opt[0, 0, 1] = 1.0
    result = harness.compare_outputs(ref, opt, 0.02, 0.002)
    assert result.failed_feature_dims == [1, 3]
    assert result.worst_index in ((0, 0, 1), (1, 2, 3))


def test_percentile_matches_linear_interpolation():
    values = [5.0, 1.0, 3.0, 2.0]
    assert harness.percentile(values, 0.9) == pytest.approx(4.4)
    assert harness.percentile([7.0], 0.9) == 7.0
    with pytest.raises(ValueError):
        harness.percentile([], 0.5)
    timing = harness.TimingResult([4.0, 1.0, 2.0])
    assert timing.median_ms == 2.0 and timing.min_ms == 1.0 and timing.mean_ms == pytest.approx(7 / 3)
    assert harness.TimingResult([4.0, 1.0, 2.0, 8.0]).median_ms == 3.0  # even count: midpoint


def test_percentile_agrees_with_numpy_linear_method():
    """numpy's default ("linear", rank q (n - 1)) percentile is the same rule; ends are min / max."""
    import numpy as np

    rng = np.random.default_rng(7)
    for n in (1, 2, 3, 10, 101):
        values = rng.exponential(size=n).tolist()
        for q in (0.0, 0.1, 0.5, 0.9, 0.99, 1.0):
            assert harness.percentile(values, q) == pytest.approx(float(np.percentile(values, 100 * q)), rel=1e-12)
        assert harness.percentile(values, 0.0) == min(values) and harness.percentile(values, 1.0) == max(values)


def test_resolve_device():
    assert harness.resolve_device("cpu") == torch.device("cpu")
    expected = "cuda" if torch.cuda.is_available() else "cpu"
    assert harness.resolve_device("auto").type == expected
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError):
            harness.resolve_device("cuda")


def test_generate_random_case_mask_and_seed():
    config = TransformerConfig(3, 10, 4, 1, 4, 1, True)
    x1, m1 = harness.generate_random_case(config, torch.device("cpu"), torch.float32, 5, 0.5, 2.0)
    x2, m2 = harness.generate_random_case(config, torch.device("cpu"), torch.float32, 5, 0.5, 2.0)
    assert torch.equal(x1, x2) and torch.equal(m1, m2)
    lengths = m1.sum(1)
    assert bool((lengths >= 5).all()) and bool((lengths <= 10).all())
    assert torch.count_nonzero(x1[~m1]) == 0
    # prefix masks: valid positions form a prefix
    for row in m1:
        n = int(row.sum())
        assert bool(row[:n].all()) and not bool(row[n:].any())


def test_microbatched_input_slices_are_independent_seeds():
    config = TransformerConfig(5, 3, 4, 1, 4, 1, True)
    x = harness.generate_microbatched_case(config, torch.device("cpu"), 77, 2)
    g = torch.Generator().manual_seed(78)
    assert torch.equal(x[2:4], torch.randn(2, 3, 4, generator=g))
    g = torch.Generator().manual_seed(79)
    assert torch.equal(x[4:5], torch.randn(1, 3, 4, generator=g))


class _Echo(torch.nn.Module):
    def forward(self, x, mask=None):
        return x * 2


class _EchoInto(torch.nn.Module):
    writes_into_out = True

    def forward(self, x, mask=None, *, out=None):
        assert out is not None and out.shape == x.shape
        out.copy_(x * 2)
        return out


def test_microbatch_wrappers_are_exact():
    x = torch.randn(7, 3, 2)
    full = _Echo()(x)
    assert torch.equal(harness.MicrobatchModel(_Echo(), 3)(x), full)
    assert torch.equal(harness.PreallocatedMicrobatchModel(_Echo(), 3)(x), full)
    # a model that writes into a given tensor receives the output's slices
    assert torch.equal(harness.PreallocatedMicrobatchModel(_EchoInto(), 3)(x), full)


def test_preallocated_microbatch_returns_a_fresh_output_per_call():
    """``mixed_precision_benchmark.py:26`` allocates the output inside forward: a caller that
    keeps two results must see both unchanged."""
    for model in (_Echo(), _EchoInto()):
        runner = harness.PreallocatedMicrobatchModel(model, 3)
        x1, x2 = torch.randn(7, 3, 2), torch.randn(7, 3, 2)
        first = runner(x1)
        second = runner(x2)
        assert first.data_ptr() != second.data_ptr()
        assert torch.equal(first, x1 * 2) and torch.equal(second, x2 * 2)


class _Wrapper(torch.nn.Module):
    """Stands in for torch.compile's wrapper, which forwards instance attribute reads."""

    def __init__(self, inner):
        super().__init__()
        self.inner = inner

    def __getattr__(self, name):
        if name == "writes_into_out":
            return getattr(self.inner, name)
        return super().__getattr__(name)

    def forward(self, x, mask=None):
        return self.inner(x, mask)


def test_preallocated_microbatch_copies_through_wrappers():
    """A wrapped module (a compiled graph) is called without ``out=``, as in the reference."""
    x = torch.randn(7, 3, 2)
    wrapped = _Wrapper(_EchoInto())
    assert wrapped.writes_into_out
    calls = []
    inner = wrapped.inner

    def forward(x, mask=None, *, out=None):
        calls.append(out is None)
        return x * 2

    inner.forward = forward
    assert torch.equal(harness.PreallocatedMicrobatchModel(wrapped, 3)(x), x * 2)
    assert calls and all(calls)
