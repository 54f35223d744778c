"""CLI argument validation and the no-GPU error path (CPU only)."""

from __future__ import annotations

import pytest
import torch

from tiktoktechjam2026_amd.mixed_precision_benchmark import main

BASE = ["--batch-size", "2", "--seq-len", "16", "--d-model", "32", "--heads", "2", "--ffn-dim", "64",
        "--layers", "1", "--causal"]


@pytest.mark.parametrize(
    "extra",
    [["--padding-ratio", "1.0"], ["--input-scale", "0"], ["--accuracy-trials", "0"], ["--repeats", "0"],
     ["--rtol", "-1"], ["--microbatch-size", "-1"], ["--warmup", "-1"]],
)
def test_invalid_arguments_raise(extra):
    with pytest.raises(ValueError):
        main(BASE + ["--device", "cpu"] + extra)


def test_invalid_config_raises():
    with pytest.raises(ValueError, match="divisible"):
        main(["--batch-size", "2", "--seq-len", "16", "--d-model", "30", "--heads", "4", "--device", "cpu"])


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU path")
def test_cpu_device_is_rejected():
    with pytest.raises(SystemExit):
        main(BASE + ["--device", "cpu"])
