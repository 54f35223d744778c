"""The benchmark CLI end to end (GPU): reference line formats and exit codes.

The strict-FP32 baseline module is injected (the oracle restatement), as the
reference CLI imports ``torch_transformer_benchmark`` for it.
"""

from __future__ import annotations

import re
import types

import pytest
import torch

from oracle import strict_fp32
from tiktoktechjam2026_amd.mixed_precision_benchmark import main

pytestmark = pytest.mark.gpu

ARGS = ["--batch-size", "4", "--seq-len", "128", "--d-model", "128", "--heads", "4", "--ffn-dim", "128",
        "--layers", "2", "--causal", "--accuracy-trials", "2", "--warmup", "2", "--repeats", "3",
        "--benchmark-rounds", "2"]


def test_cli_passes_and_prints_reference_lines(hip_device, capsys):
    rc = main(ARGS, reference=strict_fp32)
    out = capsys.readouterr().out
    assert rc == 0, out
    # the reference suite's scraping regexes (run_mixed_suite.ps1:47-53)
    assert re.search(r"summary: (PASS|FAIL)", out).group(1) == "PASS"
    assert re.search(r"summary: (?:PASS|FAIL) \| max_abs=([^|]+)", out)
    assert re.search(r"summary: (?:PASS|FAIL).*failed=([^\r\n]+)", out).group(1).strip().startswith("0/")
    assert re.search(r"baseline : median=([0-9.]+) ms", out)
    assert re.search(r"optimized: median=([0-9.]+) ms", out)
    assert re.search(r"speedup  : ([0-9.]+)x", out)
    assert "trial 01/2: PASS" in out and "trial 02/2: PASS" in out


def test_cli_cpu_baseline(hip_device, capsys):
    rc = main(ARGS + ["--baseline-device", "cpu", "--cpu-threads", "4"], reference=strict_fp32)
    out = capsys.readouterr().out
    assert rc == 0, out
    assert "baseline_device=cpu" in out


def test_cli_reports_failure_and_skips_timing(hip_device, capsys):
    """A perturbed baseline (mistake planted in the oracle, on the CPU side of the check) fails the rule."""

    class Skewed(strict_fp32.BaselineTransformer):
        def forward(self, x, valid_token_mask=None):
            return super().forward(x, valid_token_mask) + 0.01

    planted = types.SimpleNamespace(BaselineTransformer=Skewed)
    rc = main(ARGS, reference=planted)
    out = capsys.readouterr().out
    assert rc == 2
    assert "summary: FAIL" in out
    assert "Performance benchmark skipped" in out
