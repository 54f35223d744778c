"""Accuracy and timing harness (restates ``torch_transformer_benchmark.py:390-924``).

Same contracts and printed line formats as the reference harness:

* ``generate_random_case`` (:448-486) - seeded ``x ~ N(0,1)*input_scale`` and a
  prefix valid-token mask.  Deliberate difference: the generator always lives
  on the CPU and ``x`` is copied to the target device, so a CPU oracle and a
  GPU candidate see bit-identical inputs (the reference draws on the device).
* ``compare_outputs`` / ``AccuracyResult`` (:489-570) - an element passes iff
  both values are finite and ``|d| <= atol`` or ``|d| <= rtol*|ref|``.
* ``run_accuracy_tests`` (:573-638), ``percentile`` (:641-653),
  ``TimingResult`` (:656-674), ``warmup_model`` (:677-688),
  ``benchmark_once`` (:691-722), ``benchmark_models`` (:725-797).
* ``MicrobatchModel`` (:808-833) and ``PreallocatedMicrobatchModel``
  (``mixed_precision_benchmark.py:13-33``).
* ``maybe_compile`` (:800-805): on a GPU the ``reduce-overhead`` request is
  served by capturing the HIP forward into a HIP graph (``HipGraphModel``)
  instead of ``torch.compile``.
* ``parse_args`` / ``validate_args`` / ``resolve_device`` (:836-924, :415-420).

``seeded_reference_state_dict`` produces the strict-FP32 model's seeded
parameters (same draws, same order as the reference's module construction) so
benchmarks can build weights without the oracle module.
"""

from __future__ import annotations

import argparse
import math
import time
from dataclasses import dataclass
from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn


# --------------------------------------------------------------------------- weights

_LINEARS = (
    ("attention.q_proj", "d", "d"),
    ("attention.k_proj", "d", "d"),
    ("attention.v_proj", "d", "d"),
    ("attention.out_proj", "d", "d"),
    ("ffn_in", "d", "f"),
    ("ffn_out", "f", "d"),
)


def seeded_reference_state_dict(config, seed: Optional[int]) -> Dict[str, torch.Tensor]:
    """Parameters of the strict-FP32 reference model after ``torch.manual_seed(seed)``.

    Draw order per layer: q, k, v, out projections, ffn_in, ffn_out; each
    ``nn.Linear`` draws kaiming-uniform(a=sqrt(5)) weights then U(+-1/sqrt(fan_in))
    biases (``torch_transformer_benchmark.py:149-152, 205-209, 229-237``).
    LayerNorms are gamma=1, beta=0.  ``seed=None`` continues the current RNG.
    """
    if seed is not None:
        torch.manual_seed(seed)
    sizes = {"d": int(config.d_model), "f": int(config.ffn_dim)}
    d = sizes["d"]
    out: Dict[str, torch.Tensor] = {}
    for layer in range(int(config.num_layers)):
        drawn = {}
        for name, fin, fout in _LINEARS:
            lin = nn.Linear(sizes[fin], sizes[fout])  # default init draws weight, then bias
            drawn[name] = (lin.weight.detach().clone(), lin.bias.detach().clone())
        p = f"layers.{layer}."
        out[p + "norm1.weight"], out[p + "norm1.bias"] = torch.ones(d), torch.zeros(d)
        for name in ("attention.q_proj", "attention.k_proj", "attention.v_proj", "attention.out_proj"):
            out[p + name + ".weight"], out[p + name + ".bias"] = drawn[name]
        out[p + "norm2.weight"], out[p + "norm2.bias"] = torch.ones(d), torch.zeros(d)
        for name in ("ffn_in", "ffn_out"):
            out[p + name + ".weight"], out[p + name + ".bias"] = drawn[name]
    out["final_norm.weight"], out["final_norm.bias"] = torch.ones(d), torch.zeros(d)
    return out


# --------------------------------------------------------------------------- inputs


def resolve_device(device_arg: str) -> torch.device:
    """``--device`` (``torch_transformer_benchmark.py:428-434``): ``auto`` is the GPU when torch
    sees one and the CPU otherwise; naming a GPU device that torch cannot see is an error."""
    gpu_visible = torch.cuda.is_available()
    name = ("cuda" if gpu_visible else "cpu") if device_arg == "auto" else device_arg
    device = torch.device(name)
    if device.type == "cuda" and not gpu_visible:
        raise RuntimeError(f"--device {device_arg}: torch sees no GPU (torch.cuda.is_available() is False)")
    return device


def generate_random_case(
    config,
    device: torch.device,
    dtype: torch.dtype,
    seed: int,
    padding_ratio: float,
    input_scale: float,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Seeded input and valid-token mask, drawn on the CPU then moved to ``device``."""
    generator = torch.Generator(device="cpu")
    generator.manual_seed(seed)
    x = torch.randn(config.batch_size, config.seq_len, config.d_model, generator=generator, dtype=dtype)
    x = x * input_scale
    if padding_ratio <= 0:
        mask = torch.ones(config.batch_size, config.seq_len, dtype=torch.bool)
        return x.to(device), mask.to(device)
    min_valid = max(1, int(round(config.seq_len * (1.0 - padding_ratio))))
    lengths = torch.randint(
        low=min_valid, high=config.seq_len + 1, size=(config.batch_size,), generator=generator
    )
    positions = torch.arange(config.seq_len)[None, :]
    mask = positions < lengths[:, None]
    x = x.masked_fill(~mask[..., None], 0)
    return x.to(device), mask.to(device)


def generate_microbatched_case(
    config, device: torch.device, seed: int, microbatch: int, input_scale: float = 1.0
) -> torch.Tensor:
    """FP32 input whose batch slice ``i`` (of ``microbatch`` rows) is drawn from seed ``seed + i``.

    Used for the large-activation configuration so each slice can be
    regenerated independently (and on the CPU, slice by slice).
    """
    out = torch.empty(config.batch_size, config.seq_len, config.d_model, dtype=torch.float32, device=device)
    for index, start in enumerate(range(0, config.batch_size, microbatch)):
        end = min(start + microbatch, config.batch_size)
        generator = torch.Generator(device="cpu")
        generator.manual_seed(seed + index)
        chunk = torch.randn(end - start, config.seq_len, config.d_model, generator=generator) * input_scale
        out[start:end].copy_(chunk)
    return out


# --------------------------------------------------------------------------- accuracy


@dataclass
class AccuracyResult:
    """One trial of the accuracy check; the field names are those the report prints
    (``torch_transformer_benchmark.py:489-500``).  ``worst_index`` is the element of the largest
    absolute error (NaN counts as largest), ``failed_feature_dims`` the last-axis indices
    holding any failed element."""

    passed: bool
    total_elements: int
    failed_elements: int
    max_abs_error: float
    max_relative_error: float
    mean_abs_error: float
    failed_feature_dims: List[int]
    worst_index: Tuple[int, ...]
    reference_at_worst: float
    optimized_at_worst: float


def compare_outputs(reference: torch.Tensor, optimized: torch.Tensor, rtol: float, atol: float) -> AccuracyResult:
    """Element-wise rule: finite(ref) & finite(opt) & (|d| <= atol | |d| <= rtol*|ref|)."""
    if reference.shape != optimized.shape:
        raise AssertionError(
            f"shape mismatch: baseline={tuple(reference.shape)}, optimized={tuple(optimized.shape)}"
        )
    if reference.dtype != optimized.dtype:
        print(f"[warning] dtype mismatch: baseline={reference.dtype}, optimized={optimized.dtype}")
    ref = reference.detach().float()
    opt = optimized.detach().float().to(ref.device)
    finite = torch.isfinite(ref) & torch.isfinite(opt)
    abs_error = (opt - ref).abs()
    passed_mask = finite & ((abs_error <= atol) | (abs_error <= rtol * ref.abs()))
    failed_mask = ~passed_mask
    failed = int(failed_mask.sum().item())
    total = reference.numel()
    if total:
        flat_worst = int(torch.nan_to_num(abs_error, nan=float("inf")).reshape(-1).argmax().item())
    else:
        flat_worst = 0
    worst = []
    remaining = flat_worst
    for size in reversed(reference.shape):
        worst.append(remaining % size if size else 0)
        remaining //= max(size, 1)
    worst_index = tuple(reversed(worst))
    relative = abs_error / ref.abs().clamp_min(1e-12)
    if reference.ndim == 0:
        failed_dims = [0] if failed else []
    elif reference.ndim == 1:
        failed_dims = torch.nonzero(failed_mask, as_tuple=False).flatten().tolist()
    else:
        by_feature = failed_mask.any(dim=tuple(range(reference.ndim - 1)))
        failed_dims = torch.nonzero(by_feature, as_tuple=False).flatten().tolist()
    return AccuracyResult(
        passed=failed == 0,
        total_elements=total,
        failed_elements=failed,
        max_abs_error=float(abs_error.max().item()) if total else 0.0,
        max_relative_error=float(relative.max().item()) if total else 0.0,
        mean_abs_error=float(abs_error.mean().item()) if total else 0.0,
        failed_feature_dims=failed_dims,
        worst_index=worst_index,
        reference_at_worst=float(ref[worst_index].item()) if total else 0.0,
        optimized_at_worst=float(opt[worst_index].item()) if total else 0.0,
    )


def run_accuracy_tests(
    baseline: nn.Module,
    optimized: nn.Module,
    config,
    device: torch.device,
    dtype: torch.dtype,
    trials: int,
    seed: int,
    padding_ratio: float,
    input_scale: float,
    rtol: float,
    atol: float,
    baseline_device: Optional[torch.device] = None,
) -> bool:
    """Seeded trials ``seed + trial``; prints per-trial and summary lines in the reference format.

    ``baseline_device`` runs the baseline on another device (e.g. the host
    CPU) with the bit-identical input.
    """
    print("\n=== Accuracy check ===")
    print(f"criterion: abs_error <= {atol:g} OR relative_error <= {rtol:.2%}")
    all_passed = True
    max_abs = max_rel = 0.0
    total_failed = total = 0
    with torch.inference_mode():
        for trial in range(trials):
            x, mask = generate_random_case(config, device, dtype, seed + trial, padding_ratio, input_scale)
            if baseline_device is not None and baseline_device != device:
                reference = baseline(x.to(baseline_device), mask.to(baseline_device))
            else:
                reference = baseline(x, mask)
            candidate = optimized(x, mask)
            result = compare_outputs(reference, candidate.to(reference.device), rtol=rtol, atol=atol)
            all_passed &= result.passed
            max_abs = max(max_abs, result.max_abs_error)
            max_rel = max(max_rel, result.max_relative_error)
            total_failed += result.failed_elements
            total += result.total_elements
            status = "PASS" if result.passed else "FAIL"
            print(
                f"trial {trial + 1:02d}/{trials}: {status} | max_abs={result.max_abs_error:.6g} | "
                f"max_rel={result.max_relative_error:.6g} | failed={result.failed_elements}/{result.total_elements}"
            )
            if not result.passed:
                preview = result.failed_feature_dims[:16]
                suffix = "..." if len(result.failed_feature_dims) > len(preview) else ""
                print(
                    f"  worst_index={result.worst_index}, baseline={result.reference_at_worst:.8g}, "
                    f"optimized={result.optimized_at_worst:.8g}"
                )
                print(f"  failed output feature dims={preview}{suffix}")
    print(
        f"summary: {'PASS' if all_passed else 'FAIL'} | max_abs={max_abs:.6g} | max_rel={max_rel:.6g} | "
        f"failed={total_failed}/{total}"
    )
    return all_passed


# --------------------------------------------------------------------------- timing


def percentile(values: List[float], q: float) -> float:
    """The q-quantile at rank q (n - 1) of the sorted samples, interpolated linearly between
    the two order statistics around it (numpy's default method) - how the reference's report
    computes its p90 (``torch_transformer_benchmark.py:641-653``)."""
    if len(values) == 0:
        raise ValueError("values must not be empty")
    ordered = sorted(values)
    rank = q * (len(ordered) - 1)
    below = math.floor(rank)
    frac = rank - below
    if frac == 0:
        return ordered[below]
    return ordered[below] + frac * (ordered[below + 1] - ordered[below])


@dataclass
class TimingResult:
    """Per-call latencies (ms) of one timed model and the four figures the report prints from
    them: mean, median, p90 and minimum (``torch_transformer_benchmark.py:656-674``)."""

    samples_ms: List[float]

    @property
    def mean_ms(self) -> float:
        return math.fsum(self.samples_ms) / len(self.samples_ms)

    @property
    def median_ms(self) -> float:
        return percentile(self.samples_ms, 0.5)

    @property
    def p90_ms(self) -> float:
        return percentile(self.samples_ms, 0.9)

    @property
    def min_ms(self) -> float:
        return min(self.samples_ms)


def warmup_model(model: nn.Module, x: torch.Tensor, mask: torch.Tensor, iterations: int, device: torch.device) -> None:
    with torch.inference_mode():
        for _ in range(iterations):
            model(x, mask)
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def benchmark_once(
    model: nn.Module, x: torch.Tensor, mask: torch.Tensor, iterations: int, device: torch.device
) -> List[float]:
    """Per-call latency samples: HIP events on the current stream (GPU) or perf_counter_ns (CPU)."""
    samples: List[float] = []
    with torch.inference_mode():
        if device.type == "cuda":
            starts = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
            ends = [torch.cuda.Event(enable_timing=True) for _ in range(iterations)]
            torch.cuda.synchronize(device)
            for i in range(iterations):
                starts[i].record()
                model(x, mask)
                ends[i].record()
            torch.cuda.synchronize(device)
            samples.extend(s.elapsed_time(e) for s, e in zip(starts, ends))
        else:
            for _ in range(iterations):
                t0 = time.perf_counter_ns()
                model(x, mask)
                samples.append((time.perf_counter_ns() - t0) / 1e6)
    return samples


def _print_timing(label: str, result: TimingResult, tokens: int) -> None:
    tps = tokens * 1000.0 / result.median_ms
    print(
        f"{label}: median={result.median_ms:.4f} ms | mean={result.mean_ms:.4f} ms | p90={result.p90_ms:.4f} ms | "
        f"min={result.min_ms:.4f} ms | throughput={tps:.2f} token/s"
    )


def benchmark_models(
    baseline: nn.Module,
    optimized: nn.Module,
    config,
    device: torch.device,
    dtype: torch.dtype,
    seed: int,
    padding_ratio: float,
    input_scale: float,
    warmup: int,
    repeats: int,
    rounds: int,
    baseline_device: Optional[torch.device] = None,
    baseline_repeats: Optional[int] = None,
    baseline_warmup: Optional[int] = None,
) -> Tuple[TimingResult, TimingResult]:
    """Alternating-order timing of baseline and candidate on the fixed input ``seed + 100000``."""
    print("\n=== Performance benchmark ===")
    print("timing excludes random-data generation and uses a fixed input")
    if device.type == "cuda":
        print("GPU latency is measured with HIP events on the current stream")
    x, mask = generate_random_case(config, device, dtype, seed + 100000, padding_ratio, input_scale)
    bdev = baseline_device or device
    bx, bmask = x.to(bdev), mask.to(bdev)
    b_repeats = baseline_repeats or repeats
    warmup_model(baseline, bx, bmask, warmup if baseline_warmup is None else baseline_warmup, bdev)
    warmup_model(optimized, x, mask, warmup, device)
    base_samples: List[float] = []
    opt_samples: List[float] = []
    for round_index in range(rounds):
        if round_index % 2 == 0:
            base_samples.extend(benchmark_once(baseline, bx, bmask, b_repeats, bdev))
            opt_samples.extend(benchmark_once(optimized, x, mask, repeats, device))
        else:
            opt_samples.extend(benchmark_once(optimized, x, mask, repeats, device))
            base_samples.extend(benchmark_once(baseline, bx, bmask, b_repeats, bdev))
    base = TimingResult(base_samples)
    opt = TimingResult(opt_samples)
    tokens = config.batch_size * config.seq_len
    _print_timing("baseline ", base, tokens)
    _print_timing("optimized", opt, tokens)
    print(f"speedup  : {base.median_ms / opt.median_ms:.3f}x based on median latency")
    return base, opt


# --------------------------------------------------------------------------- execution wrappers


class HipGraphModel(nn.Module):
    """Replays the model's forward from a captured HIP graph (one per input shape).

    Serves the reference's ``torch.compile(mode="reduce-overhead")`` request:
    the first call for a shape warms up and captures; later calls copy ``x``
    into the static input buffer and replay.  The returned tensor is the
    graph's static output and is overwritten by the next call, as with the
    reference's compiled module.  Masked calls run eagerly.
    """

    def __init__(self, model: nn.Module) -> None:
        super().__init__()
        self.model = model
        self._graphs: Dict[tuple, tuple] = {}

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if not x.is_cuda:
            return self.model(x, valid_token_mask)
        if valid_token_mask is not None and not getattr(self.model, "assume_all_tokens_valid", False):
            return self.model(x, valid_token_mask)
        key = (tuple(x.shape), x.dtype, x.device)
        entry = self._graphs.get(key)
        if entry is None:
            static_x = x.clone()
            side = torch.cuda.Stream(device=x.device)
            side.wait_stream(torch.cuda.current_stream(x.device))
            with torch.cuda.stream(side), torch.inference_mode():
                self.model(static_x, None)  # warm-up outside the graph
            torch.cuda.current_stream(x.device).wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph), torch.inference_mode():
                static_out = self.model(static_x, None)
            entry = (graph, static_x, static_out)
            self._graphs[key] = entry
        graph, static_x, static_out = entry
        static_x.copy_(x)
        graph.replay()
        return static_out


def maybe_compile(model: nn.Module, enabled: bool, mode: str) -> nn.Module:
    """GPU: wrap in ``HipGraphModel`` (any mode); CPU: ``torch.compile`` as in the reference."""
    if not enabled:
        return model
    if torch.cuda.is_available():
        return HipGraphModel(model)
    if not hasattr(torch, "compile"):
        raise RuntimeError("this PyTorch build does not provide torch.compile")
    return torch.compile(model, mode=mode)


class MicrobatchModel(nn.Module):
    """Run independent batch slices and concatenate (caps activation memory)."""

    def __init__(self, model: nn.Module, microbatch_size: int) -> None:
        super().__init__()
        self.model = model
        self.microbatch_size = microbatch_size

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if x.shape[0] <= self.microbatch_size:
            return self.model(x, valid_token_mask)
        outputs = []
        for start in range(0, x.shape[0], self.microbatch_size):
            end = min(start + self.microbatch_size, x.shape[0])
            mask = None if valid_token_mask is None else valid_token_mask[start:end]
            outputs.append(self.model(x[start:end], mask))
        return torch.cat(outputs, dim=0)


class PreallocatedMicrobatchModel(nn.Module):
    """Microbatched forward into one FP32 output allocated per call (``mixed_precision_benchmark.py:13-33``).

    As in the reference, every call returns a tensor of its own (``torch.empty_like``, served
    by the caching allocator), so results kept from earlier calls are never overwritten."""

    def __init__(self, model: nn.Module, microbatch_size: int) -> None:
        super().__init__()
        self.model = model
        self.microbatch_size = microbatch_size

    def forward(self, x: torch.Tensor, valid_token_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        if x.shape[0] <= self.microbatch_size:
            return self.model(x, valid_token_mask)
        out = torch.empty_like(x, dtype=torch.float32)
        # A module that can write its result into a given tensor fills each slice directly (same
        # values, no copy); any other model, including a ``torch.compile`` wrapper around such a
        # module (the class attribute is looked up on the wrapper's own type, so a compiled graph
        # is never handed an output to mutate), is copied in as the reference does.
        direct = bool(getattr(type(self.model), "writes_into_out", False))
        for start in range(0, x.shape[0], self.microbatch_size):
            end = min(start + self.microbatch_size, x.shape[0])
            mask = None if valid_token_mask is None else valid_token_mask[start:end]
            if direct:
                self.model(x[start:end], mask, out=out[start:end])
            else:
                out[start:end].copy_(self.model(x[start:end], mask))
        return out


# --------------------------------------------------------------------------- command line


def build_parser(description: str) -> argparse.ArgumentParser:
    """Flags of ``torch_transformer_benchmark.py:836-905`` (same names and defaults)."""
    parser = argparse.ArgumentParser(description=description)
    parser.add_argument("--batch-size", type=int, default=8)
    parser.add_argument("--seq-len", type=int, default=128)
    parser.add_argument("--d-model", type=int, default=512)
    parser.add_argument("--heads", type=int, default=8)
    parser.add_argument("--ffn-dim", type=int, default=2048)
    parser.add_argument("--layers", type=int, default=6)
    parser.add_argument("--causal", action="store_true")
    parser.add_argument("--device", default="auto", help="auto, cpu, cuda, cuda:0, ...")
    parser.add_argument("--dtype", choices=("float32", "float16", "bfloat16"), default="float32")
    parser.add_argument("--padding-ratio", type=float, default=0.0)
    parser.add_argument("--input-scale", type=float, default=1.0)
    parser.add_argument(
        "--microbatch-size", type=int, default=None,
        help="maximum inference batch slice; defaults to 250 for GPU batches >= 4096, 0 disables",
    )
    parser.add_argument("--accuracy-trials", type=int, default=5)
    parser.add_argument("--rtol", type=float, default=0.02)
    parser.add_argument("--atol", type=float, default=0.002)
    parser.add_argument("--seed", type=int, default=1234)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--repeats", type=int, default=100)
    parser.add_argument("--benchmark-rounds", type=int, default=3)
    parser.add_argument("--benchmark-on-failure", action="store_true")
    parser.add_argument("--compile-baseline", action="store_true")
    parser.add_argument(
        "--compile-user", action=argparse.BooleanOptionalAction, default=None,
        help="capture the optimized model in a HIP graph; defaults to enabled on GPU, disabled on CPU",
    )
    parser.add_argument(
        "--compile-mode", choices=("default", "reduce-overhead", "max-autotune"), default="reduce-overhead"
    )
    parser.add_argument("--non-strict-weight-copy", action="store_true")
    parser.add_argument("--matmul-precision", choices=("highest", "high", "medium"), default="high")
    parser.add_argument(
        "--allow-tf32", action=argparse.BooleanOptionalAction, default=True,
        help="enable/disable TF32 on GPU for both implementations",
    )
    return parser


def parse_args(argv: Optional[List[str]] = None) -> argparse.Namespace:
    return build_parser("Compare a baseline and optimized PyTorch Transformer").parse_args(argv)


# Argument checks of ``torch_transformer_benchmark.py:908-922``, in its order: (the condition
# that rejects the arguments, the message the reference raises for it).
_ARG_REJECTIONS = (
    (lambda a: not 0.0 <= a.padding_ratio < 1.0, "padding_ratio must be in [0, 1)"),
    (lambda a: a.input_scale <= 0, "input_scale must be positive"),
    (lambda a: a.microbatch_size is not None and a.microbatch_size < 0, "microbatch_size must be non-negative"),
    (lambda a: a.accuracy_trials <= 0, "accuracy_trials must be positive"),
    (lambda a: a.rtol < 0 or a.atol < 0, "rtol and atol must be non-negative"),
    (lambda a: a.warmup < 0, "warmup must be non-negative"),
    (lambda a: a.repeats <= 0 or a.benchmark_rounds <= 0, "repeats and benchmark_rounds must be positive"),
)


def validate_args(args: argparse.Namespace, device: torch.device, dtype: torch.dtype) -> None:
    """Raise ``ValueError`` with the first rejection that applies; warn about FP16 on the CPU."""
    for rejects, message in _ARG_REJECTIONS:
        if rejects(args):
            raise ValueError(message)
    if device.type == "cpu" and dtype == torch.float16:
        print("[warning] float16 CPU kernels may be unsupported or slow")
