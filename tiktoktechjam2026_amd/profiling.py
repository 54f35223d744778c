"""Per-kernel timing and roofline accounting for the HIP forward.

``forward_kernel_table`` times every distinct kernel launch of one forward
(row-fused route: initial LayerNorm, QKV projection, attention,
out-projection + LN, FFN + LN; GEMM route: LayerNorm, QKV projection,
attention, out-projection + residual, FFN-in + GELU, FFN-out + residual;
layer-tail route: LayerNorm + QKV, attention, layer tail, last-layer tail) in
isolation with HIP events recorded on the stream the kernel is launched on
(torch's current stream, which is the stream the C ABI is given), and prices
each against its algorithmic work:

* projection ``Y = X W^T + b``:   FLOPs 2MNK;  bytes M K s_in + N K 2 + N 2 + M N s_out
* projection + residual (FP32):   FLOPs 2MNK;  bytes M K 2 + N K 2 + N 2 + 8 M N
* out-projection + residual + LN: FLOPs 2 M D^2; bytes M D s_in + 2 D^2 + 8 M D + M D s_norm + 16 D
* FFN + residual + LN:            FLOPs 4 M D F; bytes M D s_in + 4 D F + M D (8 + s_norm)
* causal attention:               FLOPs 2 B H hd S (S+1); bytes 8 B S D (fp16 q, k, v in, o out)
* LayerNorm (no residual):        bytes M D (4 + s_norm)
* LayerNorm + QKV:                FLOPs 6 M D^2; bytes 4 M D + 6 M D + 6 D^2
* layer tail (to the next QKV):   FLOPs 8 M D^2 + 4 M D F; bytes M D (2 + 4 + 4 + 6) + 2 (4 D^2 + 2 D F)
* last-layer tail (final LN out): FLOPs 2 M D^2 + 4 M D F; bytes 14 M D + 2 (D^2 + 2 D F)

(s_* = bytes per element).  The binding roof of a kernel is the larger of
FLOPs / MFMA peak and bytes / HBM peak; ``frac`` is achieved / peak on that roof.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Dict, List

import torch

# MI355X published peaks (dense).
PEAK_FP16_MFMA_FLOPS = 2.5e15
PEAK_HBM_BYTES = 8.0e12


@dataclass
class KernelCost:
    name: str
    launches_per_forward: int
    flops: float
    bytes: float

    @property
    def bound(self) -> str:
        return "mfma" if self.flops / PEAK_FP16_MFMA_FLOPS >= self.bytes / PEAK_HBM_BYTES else "hbm"


def forward_costs(config, normalized_bytes: int = 2, route=None) -> Dict[str, KernelCost]:
    """Algorithmic FLOPs / bytes per launch of each kernel of one forward (one microbatch).

    ``route`` is a ``dispatch.Route`` (default: the route ``dispatch.plan`` picks
    for ``config``); only the kernels that route launches are listed.
    """
    from . import dispatch

    if route is None:
        route = dispatch.plan(config)
    B, S, D = int(config.batch_size), int(config.seq_len), int(config.d_model)
    H, F, L = int(config.num_heads), int(config.ffn_dim), int(config.num_layers)
    M = B * S
    hd = D // H
    sn = normalized_bytes
    pairs = S * (S + 1) / 2 if config.causal else S * S
    attention = KernelCost("attention", L, 4.0 * B * H * hd * pairs, 8.0 * B * S * D)
    if route.fuse_layer_tail:
        w_tail = 2.0 * (D * D + 2 * D * F + 3 * D * D)
        return {
            "layernorm_qkv": KernelCost(
                "layernorm_qkv", 1, 2.0 * M * 3 * D * D, M * D * 4 + M * 3 * D * 2 + 2.0 * 3 * D * D
            ),
            "attention": attention,
            "layer_tail": KernelCost(
                "layer_tail", L - 1, 2.0 * M * D * D + 4.0 * M * D * F + 6.0 * M * D * D,
                M * D * (2 + 4 + 4) + M * 3 * D * 2 + w_tail,
            ),
            "layer_tail_last": KernelCost(
                "layer_tail_last", 1, 2.0 * M * D * D + 4.0 * M * D * F,
                M * D * (2 + 4 + 4 + 4) + 2.0 * (D * D + 2 * D * F),
            ),
        }
    wide_ln = getattr(route, "wide_ln_epilogue", False)
    norm_launches = 1 if wide_ln else (
        1 + (0 if route.fuse_attention_output_norm else L) + (0 if route.fuse_full_ffn else L)
    )
    costs = {
        "layernorm": KernelCost("layernorm", norm_launches, 0.0, M * D * (4 + sn)),
        "qkv_proj": KernelCost("qkv_proj", L, 2.0 * M * 3 * D * D, M * D * sn + 3 * D * D * 2 + 3 * D * 2 + M * 3 * D * 2),
        "attention": attention,
    }
    if wide_ln:
        # residual projections with the next LayerNorm in the epilogue (256 x 256 GEMM tiles)
        costs["out_proj_ln"] = KernelCost(
            "out_proj_ln", L, 2.0 * M * D * D, M * D * 2 + 2 * D * D + 2 * D + 8 * M * D + M * D * sn + 8 * D
        )
    elif route.fuse_attention_output_norm:
        costs["out_proj_ln"] = KernelCost(
            "out_proj_ln", L, 2.0 * M * D * D, M * D * 2 + 2 * D * D + 8 * M * D + M * D * sn + 16 * D
        )
    else:
        costs["out_proj_residual"] = KernelCost(
            "out_proj_residual", L, 2.0 * M * D * D, M * D * 2 + 2 * D * D + 2 * D + 8 * M * D
        )
    if route.fuse_full_ffn:
        costs["ffn_ln"] = KernelCost("ffn_ln", L, 4.0 * M * D * F, M * D * sn + 4 * D * F + M * D * (8 + sn))
    elif wide_ln:
        costs["ffn_in"] = KernelCost("ffn_in", L, 2.0 * M * D * F, M * D * sn + 2 * D * F + 2 * F + M * F * 2)
        # the last layer's normalized output is FP32 (counted at the stream width here)
        costs["ffn_out_ln"] = KernelCost(
            "ffn_out_ln", L, 2.0 * M * D * F, M * F * 2 + 2 * D * F + 2 * D + 8 * M * D + M * D * sn + 8 * D
        )
    else:
        costs["ffn_in"] = KernelCost("ffn_in", L, 2.0 * M * D * F, M * D * sn + 2 * D * F + 2 * F + M * F * 2)
        costs["ffn_out_residual"] = KernelCost(
            "ffn_out_residual", L, 2.0 * M * D * F, M * F * 2 + 2 * D * F + 2 * D + 8 * M * D
        )
    return costs


def time_launches(fn: Callable[[], object], iterations: int, warmup: int = 3) -> float:
    """Average device duration (seconds) of one ``fn`` launch.

    ``iterations`` launches are captured into one HIP graph (so host launch
    overhead cannot hide in the figure) and the graph replay is bracketed by
    HIP events on the current stream - the stream the C ABI launches on.
    """
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iterations):
            fn()
    graph.replay()  # warm the captured sequence once
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    graph.replay()
    end.record(stream)
    end.synchronize()
    seconds = start.elapsed_time(end) / 1e3 / iterations
    del graph
    return seconds


def _row(name: str, cost: KernelCost, seconds: float) -> Dict[str, object]:
    if cost.bound == "mfma":
        achieved, peak, unit = cost.flops / seconds / 1e12, PEAK_FP16_MFMA_FLOPS / 1e12, "TFLOP/s"
    else:
        achieved, peak, unit = cost.bytes / seconds / 1e9, PEAK_HBM_BYTES / 1e9, "GB/s"
    return {
        "kernel": name,
        "launches_per_forward": cost.launches_per_forward,
        "avg_us": seconds * 1e6,
        "share_us_per_forward": seconds * 1e6 * cost.launches_per_forward,
        "bound": cost.bound,
        "achieved": achieved,
        "peak": peak,
        "unit": unit,
        "frac": achieved / peak,
        "flops": cost.flops,
        "bytes": cost.bytes,
        "tflops": cost.flops / seconds / 1e12,
        "gbps": cost.bytes / seconds / 1e9,
    }


def forward_kernel_table(model, x: torch.Tensor, iterations: int = 50) -> List[Dict[str, object]]:
    """Time each distinct kernel of ``model``'s forward on input ``x`` (first layer's weights)."""
    from .custom_kernel.hip_attention import attention
    from .mixed_precision.hip_fused import fused_layer_tail, layer_norm_qkv
    from .mixed_precision.hip_linear import (
        layer_norm, mixed_ffn_add_layer_norm, mixed_linear, mixed_linear_add_layer_norm, mixed_linear_residual,
        mixed_linear_residual_layer_norm,
    )

    import dataclasses

    route = model.route
    layer = model.layers[0]
    att = layer.attention
    B, S, D = x.shape
    # price the launches actually timed: one microbatch of B sequences
    config = dataclasses.replace(model.config, batch_size=B) if dataclasses.is_dataclass(model.config) else model.config
    sdt = route.normalized_dtype
    causal = bool(config.causal)
    costs = forward_costs(config, 2 if sdt == torch.float16 else 4, route)
    with torch.inference_mode():
        if route.fuse_layer_tail:
            qkv = layer_norm_qkv(x, layer.norm1, att.qkv_proj, variant=route.head_variant)
            q, k, v = qkv.view(B, S, 3, att.num_heads, att.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
            ctx = attention(q, k, v, att.scale, causal=causal, variant=route.attention_variant).view(B, S, D)
            launches = {
                "layernorm_qkv": lambda: layer_norm_qkv(x, layer.norm1, att.qkv_proj, variant=route.head_variant),
                "attention": lambda: attention(q, k, v, att.scale, causal=causal, variant=route.attention_variant),
                "layer_tail": lambda: fused_layer_tail(ctx, x, att.out_proj, layer.norm2, layer.ffn_in, layer.ffn_out,
                                                       layer.norm1, att.qkv_proj, variant=route.tail_variant),
                "layer_tail_last": lambda: fused_layer_tail(ctx, x, att.out_proj, layer.norm2, layer.ffn_in,
                                                            layer.ffn_out, model.final_norm, None,
                                                            variant=route.tail_variant),
            }
        else:
            normalized = layer_norm(x, layer.norm1, normalized_dtype=sdt)
            qkv = mixed_linear(normalized, att.qkv_proj, output_dtype=torch.float16, variant=route.qkv_variant)
            q, k, v = qkv.view(B, S, 3, att.num_heads, att.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
            ctx = attention(q, k, v, att.scale, causal=causal, variant=route.attention_variant).view(B, S, D)
            if route.wide_ln_epilogue:
                resid, nffn = mixed_linear_residual_layer_norm(ctx, att.out_proj, x, layer.norm2,
                                                               normalized_dtype=sdt)
            elif route.fuse_attention_output_norm:
                resid, nffn = mixed_linear_add_layer_norm(ctx, att.out_proj, x, layer.norm2, normalized_dtype=sdt,
                                                          variant=route.out_ln_variant)
            else:
                resid = mixed_linear_residual(ctx, att.out_proj, x, variant=route.out_proj_variant)
                nffn = layer_norm(resid, layer.norm2, normalized_dtype=sdt)
            hidden = mixed_linear(nffn, layer.ffn_in, output_dtype=torch.float16, fuse_gelu=True,
                                  variant=route.ffn_in_variant)
            launches = {
                "layernorm": lambda: layer_norm(x, layer.norm1, normalized_dtype=sdt),
                "qkv_proj": lambda: mixed_linear(normalized, att.qkv_proj, output_dtype=torch.float16,
                                                 variant=route.qkv_variant),
                "attention": lambda: attention(q, k, v, att.scale, causal=causal, variant=route.attention_variant),
                "out_proj_ln": (
                    (lambda: mixed_linear_residual_layer_norm(ctx, att.out_proj, x, layer.norm2, normalized_dtype=sdt))
                    if route.wide_ln_epilogue else
                    (lambda: mixed_linear_add_layer_norm(ctx, att.out_proj, x, layer.norm2, normalized_dtype=sdt,
                                                         variant=route.out_ln_variant))
                ),
                "out_proj_residual": lambda: mixed_linear_residual(ctx, att.out_proj, x,
                                                                   variant=route.out_proj_variant),
                "ffn_ln": lambda: mixed_ffn_add_layer_norm(nffn, layer.ffn_in, layer.ffn_out, resid, layer.norm1,
                                                           normalized_dtype=sdt, variant=route.ffn_variant),
                "ffn_in": lambda: mixed_linear(nffn, layer.ffn_in, output_dtype=torch.float16, fuse_gelu=True,
                                               variant=route.ffn_in_variant),
                "ffn_out_residual": lambda: mixed_linear_residual(hidden, layer.ffn_out, resid,
                                                                  variant=route.ffn_out_variant),
                "ffn_out_ln": lambda: mixed_linear_residual_layer_norm(hidden, layer.ffn_out, resid, layer.norm1,
                                                                       normalized_dtype=sdt),
            }
        rows = []
        for name, fn in launches.items():
            if name not in costs or costs[name].launches_per_forward == 0:
                continue
            rows.append(_row(name, costs[name], time_launches(fn, iterations)))
    return rows


def forward_roofline_seconds(config, microbatches: int = 1, route=None) -> float:
    """Lower bound on one forward: sum over kernels of max(FLOPs/MFMA peak, bytes/HBM peak)."""
    total = 0.0
    for cost in forward_costs(config, 2, route).values():
        total += cost.launches_per_forward * max(cost.flops / PEAK_FP16_MFMA_FLOPS, cost.bytes / PEAK_HBM_BYTES)
    return total * microbatches


def describe_rate(value: float) -> str:
    if not math.isfinite(value):
        return "n/a"
    return f"{value:,.0f}"


# --------------------------------------------------------------------------- PMC traffic helpers
#
#   python -m tiktoktechjam2026_amd.profiling run --config cfg2 --iters 3
#       runs the configured forward eagerly (no graphs) for PMC collection, after a plain
#       device copy of 1 GiB (the calibration kernel: 1 GiB read + 1 GiB written).
#   python -m tiktoktechjam2026_amd.profiling summarize FETCH.csv WRITE.csv --config cfg2 --out J
#       turns two rocprofv3 --pmc counter CSVs (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch)
#       into HBM bytes per launch per kernel, each counter scaled by copy_bytes / counter(copy).

_KERNEL_KEYS = (
    ("layer_tail_kernel<128, 32, 1, false", "layernorm_qkv"),
    ("layer_tail_kernel", "layer_tail"),
    ("attention32_kernel", "attention"),
    ("attention_kernel", "attention"),
    ("linear_big_kernel", "linear"),
    ("linear_kernel", "linear"),
    ("ffn_ln_kernel", "ffn_ln"),
    ("residual_layernorm_kernel", "layernorm"),
)
CALIBRATION_BYTES = 1 << 30


def _kernel_key(name: str) -> str:
    if "layer_tail_kernel" in name and ", true, true," in name:
        return "layer_tail_last"
    for pattern, key in _KERNEL_KEYS:
        if pattern in name:
            return key
    if "copyBuffer" in name or "copy_kernel" in name or "elementwise_kernel" in name:
        return "copy"
    return name[:60]


def _run(config_name: str, iters: int) -> None:
    from .config import BENCHMARK_CONFIGS
    from . import harness
    from .mixed_precision import MixedPrecisionTransformer, copy_mixed_model_weights

    dev = torch.device("cuda:0")
    src = torch.empty(CALIBRATION_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)  # calibration kernel
    torch.cuda.synchronize()
    del src, dst
    config = BENCHMARK_CONFIGS[config_name]
    if config.batch_size * config.seq_len > 262144:
        import dataclasses

        config = dataclasses.replace(config, batch_size=262144 // config.seq_len)
    model = MixedPrecisionTransformer(config)
    copy_mixed_model_weights(harness.seeded_reference_state_dict(config, 1234), model)
    model = model.to(dev).eval()
    model.convert_projections_to_fp16()
    x, _ = harness.generate_random_case(config, dev, torch.float32, 1234 + 100000, 0.0, 1.0)
    with torch.inference_mode():
        for _ in range(iters):
            model(x)
    torch.cuda.synchronize()


def _summarize(fetch_csv: str, write_csv: str, config_name: str, out: str) -> None:
    import csv
    import json
    from collections import defaultdict

    def per_kernel(path: str, counter: str):
        sums, counts, peak = defaultdict(float), defaultdict(int), defaultdict(float)
        with open(path) as handle:
            for row in csv.DictReader(handle):
                if row["Counter_Name"] != counter:
                    continue
                key = _kernel_key(row["Kernel_Name"])
                value = float(row["Counter_Value"])
                sums[key] += value
                counts[key] += 1
                peak[key] = max(peak[key], value)
        out = {k: sums[k] / counts[k] for k in sums}
        if "copy" in peak:
            out["copy"] = peak["copy"]  # the 1 GiB calibration copy is the largest copy dispatch
        return out

    fetch = per_kernel(fetch_csv, "FETCH_SIZE")
    write = per_kernel(write_csv, "WRITE_SIZE")
    # the calibration copy is the largest "copy" dispatch; its counters should read 1 GiB each
    f_scale = CALIBRATION_BYTES / (fetch["copy"] * 1024.0) if fetch.get("copy") else 1.0
    w_scale = CALIBRATION_BYTES / (write["copy"] * 1024.0) if write.get("copy") else 1.0
    table = {"calibration": {"copy_bytes": CALIBRATION_BYTES, "fetch_scale": f_scale, "write_scale": w_scale}}
    entry = {}
    for key in sorted(set(fetch) | set(write)):
        if key == "copy":
            continue
        fb = fetch.get(key, 0.0) * 1024.0 * f_scale
        wb = write.get(key, 0.0) * 1024.0 * w_scale
        entry[key] = {"fetch_bytes": fb, "write_bytes": wb, "bytes_per_launch": fb + wb}
    table[config_name] = entry
    try:
        with open(out) as handle:
            old = json.load(handle)
    except (OSError, ValueError):
        old = {}
    old.update(table)
    with open(out, "w") as handle:
        json.dump(old, handle, indent=1, sort_keys=True)
    print(json.dumps(table, indent=1))


if __name__ == "__main__":
    import argparse

    parser = argparse.ArgumentParser()
    sub = parser.add_subparsers(dest="cmd", required=True)
    p_run = sub.add_parser("run")
    p_run.add_argument("--config", default="cfg2")
    p_run.add_argument("--iters", type=int, default=3)
    p_sum = sub.add_parser("summarize")
    p_sum.add_argument("fetch_csv")
    p_sum.add_argument("write_csv")
    p_sum.add_argument("--config", default="cfg2")
    p_sum.add_argument("--out", default="profiles/hbm_traffic.json")
    args = parser.parse_args()
    if args.cmd == "run":
        _run(args.config, args.iters)
    else:
        _summarize(args.fetch_csv, args.write_csv, args.config, args.out)
