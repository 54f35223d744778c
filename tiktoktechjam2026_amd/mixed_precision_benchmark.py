"""Command line: strict-FP32 baseline vs the HIP mixed FP16/FP32 candidate.

Restates the reference CLI ``mixed_precision_benchmark.py:36-147`` with the same
flags (``torch_transformer_benchmark.py:836-905``), the same printed lines
(dispatch flags, ``trial NN/NN: PASS | max_abs=...``, ``summary: ...``,
``baseline : median=...``, ``optimized: median=...``, ``speedup  : ...``) and the
same exit codes (0 on pass, 2 when accuracy fails and timing is skipped), so the
reference's suite scraper (``run_mixed_suite.ps1:47-53``) parses its output.

    python -m tiktoktechjam2026_amd.mixed_precision_benchmark --batch-size 64 \
        --d-model 128 --heads 4 --seq-len 1024 --ffn-dim 128 --layers 4 --causal

The strict-FP32 baseline is the reference's own untouched module
(``torch_transformer_benchmark.BaselineTransformer``, importable when this runs
from the reference checkout); ``main(argv, reference=module)`` accepts any module
exposing ``BaselineTransformer(config)`` with the same construction-order RNG use.

Additions: ``--baseline-device cpu`` runs the baseline on the host CPU
(``--cpu-threads`` threads) against the bit-identical input, and ``--json-out``
writes the measured numbers.  ``--compile-user`` (default on GPU) captures the
candidate in a HIP graph.
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
from typing import List, Optional

import torch

from . import harness
from .config import TransformerConfig
from .mixed_precision import MixedPrecisionTransformer, copy_mixed_model_weights


def _parse(argv: Optional[List[str]]) -> argparse.Namespace:
    parser = harness.build_parser("Compare a strict-FP32 baseline with the HIP mixed FP16/FP32 candidate")
    parser.add_argument("--baseline-device", default="same", help="'same' (default) or a device such as 'cpu'")
    parser.add_argument("--cpu-threads", type=int, default=0, help="torch CPU threads for a CPU baseline")
    parser.add_argument("--json-out", default=None)
    return parser.parse_args(argv)


def _load_reference(reference):
    if reference is not None:
        return reference
    try:
        return importlib.import_module("torch_transformer_benchmark")
    except ImportError as exc:  # pragma: no cover - depends on the caller's tree
        raise SystemExit(
            "the strict-FP32 baseline module 'torch_transformer_benchmark' is not importable; run from the "
            "reference checkout (or pass reference=... to main())"
        ) from exc


def main(argv: Optional[List[str]] = None, reference=None) -> int:
    args = _parse(argv)
    device = harness.resolve_device(args.device)
    config = TransformerConfig(
        batch_size=args.batch_size,
        seq_len=args.seq_len,
        d_model=args.d_model,
        num_heads=args.heads,
        ffn_dim=args.ffn_dim,
        num_layers=args.layers,
        causal=args.causal,
    )
    config.validate()
    harness.validate_args(args, device, torch.float32)
    if device.type != "cuda":
        raise SystemExit("the HIP candidate needs a GPU device (--device cuda)")
    ref = _load_reference(reference)
    baseline_device = device if args.baseline_device == "same" else torch.device(args.baseline_device)
    if baseline_device.type == "cpu" and args.cpu_threads > 0:
        torch.set_num_threads(args.cpu_threads)

    # Strict IEEE FP32 for the baseline, regardless of the dtype/TF32 flags.
    torch.manual_seed(args.seed)
    torch.set_float32_matmul_precision("highest")
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    try:
        torch.backends.mkldnn.matmul.fp32_precision = "ieee"
    except (AttributeError, RuntimeError):
        pass
    if device.type == "cuda":
        torch.cuda.manual_seed_all(args.seed)

    baseline = ref.BaselineTransformer(config)
    mixed = MixedPrecisionTransformer(config)
    mixed.assume_all_tokens_valid = args.padding_ratio <= 0
    copy_mixed_model_weights(baseline, mixed)
    baseline = baseline.to(device=baseline_device, dtype=torch.float32).eval()
    mixed = mixed.to(device=device).eval()
    mixed.convert_projections_to_fp16()
    route = mixed.dispatch_report()

    baseline_micro = args.microbatch_size
    mixed_micro = args.microbatch_size
    if args.microbatch_size is None:
        automatic = config.batch_size >= 4096
        baseline_micro = 250 if automatic else 0
        mixed_micro = 64 if automatic else 0
    compile_mixed = args.compile_user if args.compile_user is not None else True
    baseline_model: torch.nn.Module = harness.maybe_compile(baseline, args.compile_baseline, args.compile_mode) \
        if baseline_device.type == "cuda" else baseline
    mixed_model: torch.nn.Module = harness.maybe_compile(mixed, compile_mixed, args.compile_mode)
    if baseline_micro:
        baseline_model = harness.MicrobatchModel(baseline_model, baseline_micro)
    if mixed_micro:
        mixed_model = harness.PreallocatedMicrobatchModel(mixed_model, mixed_micro)

    print("=== Strict-FP32 baseline vs mixed candidate ===")
    print(config)
    print(f"device={device}, baseline_device={baseline_device}, baseline_dtype=torch.float32, baseline_tf32=False")
    print("mixed_policy=FP16 projections; FP32 accumulation/reductions/GELU/residual/LayerNorm/output")
    print(f"case8_custom_triton_projections={mixed.use_case8_triton}")
    print(f"d128_custom_triton_projections={mixed.use_d128_triton}")
    print(f"d32_custom_triton_projections={mixed.use_d32_triton}")
    print(f"d128_custom_triton_attention={mixed.use_d128_custom_attention}")
    print(f"fp16_custom_triton_attention={mixed.use_fp16_custom_attention}")
    print(f"case11_expanded_d128_schedule={mixed.use_case11_schedule}")
    print(f"attention_output_norm_fusion={mixed.fuse_attention_output_norm}")
    print(f"full_ffn_fusion={mixed.fuse_full_ffn}")
    print(f"fp16_normalized_stream={mixed.use_fp16_normalized_stream}")
    print(f"hip_route={json.dumps(route, sort_keys=True)}")
    print(f"compile_baseline={args.compile_baseline}, compile_mixed={compile_mixed}, compile_mode=hip-graph")
    print(f"baseline_microbatch_size={baseline_micro or 'disabled'}")
    print(f"mixed_microbatch_size={mixed_micro or 'disabled'}")
    print(f"gpu={torch.cuda.get_device_name(device)}")
    if baseline_device.type == "cpu":
        print(f"baseline_cpu_threads={torch.get_num_threads()}")

    passed = harness.run_accuracy_tests(
        baseline_model, mixed_model, config, device, torch.float32, args.accuracy_trials, args.seed,
        args.padding_ratio, args.input_scale, args.rtol, args.atol, baseline_device=baseline_device,
    )
    record = {"config": config.__dict__, "accuracy_passed": passed, "route": route}
    if not passed and not args.benchmark_on_failure:
        print("\nPerformance benchmark skipped because accuracy validation failed.")
        _write(args.json_out, record)
        return 2
    base_t, opt_t = harness.benchmark_models(
        baseline_model, mixed_model, config, device, torch.float32, args.seed, args.padding_ratio, args.input_scale,
        args.warmup, args.repeats, args.benchmark_rounds, baseline_device=baseline_device,
    )
    tokens = config.batch_size * config.seq_len
    record.update(
        baseline_median_ms=base_t.median_ms,
        candidate_median_ms=opt_t.median_ms,
        candidate_tokens_per_s=tokens * 1000.0 / opt_t.median_ms,
        speedup=base_t.median_ms / opt_t.median_ms,
    )
    _write(args.json_out, record)
    return 0 if passed else 2


def _write(path: Optional[str], record: dict) -> None:
    if path:
        with open(path, "w") as handle:
            json.dump(record, handle, indent=1, default=str)


if __name__ == "__main__":
    sys.exit(main())
