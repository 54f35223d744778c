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
import os
import re
from dataclasses import dataclass
from typing import Callable, Dict, List, Optional

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
    if route.fuse_layer_tail and dispatch.attention_tail_for(route, S, masked=False):
        # attention inside the tail: per token the packed QKV (6 D) and x (4 D) are read and
        # x' (4 D) and the next QKV (6 D) - or the final normalized row (4 D) - written
        w_tail = 2.0 * (D * D + 2 * D * F + 3 * D * D)
        return {
            "layernorm_qkv": KernelCost(
                "layernorm_qkv", 1, 2.0 * M * 3 * D * D, M * D * 4 + M * 3 * D * 2 + 2.0 * 3 * D * D
            ),
            "attention_layer_tail": KernelCost(
                "attention_layer_tail", L - 1,
                attention.flops + 2.0 * M * D * D + 4.0 * M * D * F + 6.0 * M * D * D,
                M * D * (6 + 4 + 4 + 6) + w_tail,
            ),
            "attention_layer_tail_last": KernelCost(
                "attention_layer_tail_last", 1, attention.flops + 2.0 * M * D * D + 4.0 * M * D * F,
                M * D * (6 + 4 + 4 + 4) + 2.0 * (D * D + 2 * D * F),
            ),
        }
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
    wide_ln_ffn = getattr(route, "wide_ln_ffn_out", False)
    norm_launches = (
        1 + (0 if route.fuse_attention_output_norm or wide_ln else L)
        + (0 if route.fuse_full_ffn or wide_ln_ffn else L)
    )
    costs = {
        "layernorm": KernelCost("layernorm", norm_launches, 0.0, M * D * (4 + sn)),
        "qkv_proj": KernelCost("qkv_proj", L, 2.0 * M * 3 * D * D, M * D * sn + 3 * D * D * 2 + 3 * D * 2 + M * 3 * D * 2),
        "attention": attention,
    }
    if wide_ln:
        # residual projection with the next LayerNorm in the epilogue (tiles of whole rows)
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
    elif wide_ln_ffn:
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
    from .custom_kernel.hip_attention import attention, attention_prescaled
    from .mixed_precision.hip_fused import fused_attention_layer_tail, fused_layer_tail, layer_norm_qkv
    from .mixed_precision.hip_linear import (
        layer_norm, mixed_ffn_add_layer_norm, mixed_linear, mixed_linear_add_layer_norm, mixed_linear_q_scaled,
        mixed_linear_residual, mixed_linear_residual_layer_norm,
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
    from . import dispatch

    with torch.inference_mode():
        if route.fuse_layer_tail and dispatch.attention_tail_for(route, S, masked=False):
            qkv = layer_norm_qkv(x, layer.norm1, att.qkv_proj, variant=route.head_variant)
            launches = {
                "layernorm_qkv": lambda: layer_norm_qkv(x, layer.norm1, att.qkv_proj, variant=route.head_variant),
                "attention_layer_tail": lambda: fused_attention_layer_tail(
                    qkv, x, att.num_heads, att.scale, causal, att.out_proj, layer.norm2, layer.ffn_in, layer.ffn_out,
                    layer.norm1, att.qkv_proj),
                "attention_layer_tail_last": lambda: fused_attention_layer_tail(
                    qkv, x, att.num_heads, att.scale, causal, att.out_proj, layer.norm2, layer.ffn_in, layer.ffn_out,
                    model.final_norm, None),
            }
        elif route.fuse_layer_tail:
            # the route's QKV producers fold scale * log2(e) into q where the attention takes it
            qs = att.q_prescale if dispatch.prescaled_attention_for(route, S) else None
            qkv = layer_norm_qkv(x, layer.norm1, att.qkv_proj, variant=route.head_variant, q_scale=qs)
            q, k, v = qkv.view(B, S, 3, att.num_heads, att.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
            if qs is None:
                attend = lambda: attention(  # noqa: E731
                    q, k, v, att.scale, causal=causal, variant=route.attention_variant)
            else:
                attend = lambda: attention_prescaled(  # noqa: E731
                    q, k, v, causal=causal, variant=route.attention_variant)
            ctx = attend().view(B, S, D)
            launches = {
                "layernorm_qkv": lambda: layer_norm_qkv(x, layer.norm1, att.qkv_proj, variant=route.head_variant,
                                                        q_scale=qs),
                "attention": attend,
                "layer_tail": lambda: fused_layer_tail(ctx, x, att.out_proj, layer.norm2, layer.ffn_in, layer.ffn_out,
                                                       layer.norm1, att.qkv_proj, variant=route.tail_variant,
                                                       q_scale=qs),
                "layer_tail_last": lambda: fused_layer_tail(ctx, x, att.out_proj, layer.norm2, layer.ffn_in,
                                                            layer.ffn_out, model.final_norm, None,
                                                            variant=route.tail_variant),
            }
        else:
            normalized = layer_norm(x, layer.norm1, normalized_dtype=sdt)
            if dispatch.prescaled_attention_for(route, S):
                # the route's pair: q scaled by the projection, attention without a scale
                project = lambda: mixed_linear_q_scaled(  # noqa: E731
                    normalized, att.qkv_proj, D, att.q_prescale, variant=route.qkv_variant)
                qkv = project()
                q, k, v = qkv.view(B, S, 3, att.num_heads, att.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
                attend = lambda: attention_prescaled(  # noqa: E731
                    q, k, v, causal=causal, variant=route.attention_variant)
            else:
                project = lambda: mixed_linear(  # noqa: E731
                    normalized, att.qkv_proj, output_dtype=torch.float16, variant=route.qkv_variant)
                qkv = project()
                q, k, v = qkv.view(B, S, 3, att.num_heads, att.head_dim).permute(2, 0, 3, 1, 4).unbind(0)
                attend = lambda: attention(  # noqa: E731
                    q, k, v, att.scale, causal=causal, variant=route.attention_variant)
            ctx = attend().view(B, S, D)
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
                "qkv_proj": project,
                "attention": attend,
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


# --------------------------------------------------------------------------- rocprofv3 summaries
#
# Every figure in the committed profile pages comes from these commands (run from the repository
# root; the rocprofv3 output directories are written by the GPU runs):
#
#   python -m tiktoktechjam2026_amd.profiling run --config cfgN [--iters 3]
#       the configured forward, eagerly (no graphs), for counter passes: first a plain 1 GiB
#       device copy (the calibration kernel, 1 GiB read + 1 GiB written), then the forwards.
#   python -m tiktoktechjam2026_amd.profiling traffic FETCH_DIR WRITE_DIR --config cfgN
#       two `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of `run` -> HBM bytes per
#       launch per kernel (KiB per dispatch, each counter scaled by the calibration copy's
#       bytes / the counter's reading for it), merged into profiles/hbm_traffic.json.
#   python -m tiktoktechjam2026_amd.profiling mfma MFMA_DIR TRACE_DIR --config cfgN
#       one `rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 GRBM_GUI_ACTIVE
#       SQ_BUSY_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA` run of `run`, plus the kernel trace of the
#       bench command for durations -> MFMA busy fraction and counted MFMA FLOP/s per kernel,
#       merged into profiles/mfma_counters.json.
#   python -m tiktoktechjam2026_amd.profiling table RUNS_DIR
#       bench lines RUNS_DIR/bench_cfgN.json, kernel traces RUNS_DIR/prof_cfgN/ and the two
#       counter files -> profiles/forward_all_configs_mi355x.md.
#   python -m tiktoktechjam2026_amd.profiling parity-table RECORDS.json
#       whole-output parity records (tests/test_parity_full_gpu.py) ->
#       profiles/parity_all_configs_mi355x.md.

CALIBRATION_BYTES = 1 << 30
SIMD_PER_GPU = 1024  # MI355X: 256 CUs x 4 SIMDs (rocprofv3 agent info Simd_Count)
# rocprofv3 reports GRBM_GUI_ACTIVE summed over the 8 XCDs of the MI355X (each XCD
# counts the kernel's busy cycles on its own clock domain), so one kernel-duration
# worth of cycles is GRBM_GUI_ACTIVE / 8.
XCD_PER_GPU = 8

_MANGLED_ARG = re.compile(r"Li(-?\d+)E|Lb([01])E|(DF16_)|(f)|(E)")


def parse_kernel_name(name: str):
    """(base name, template arguments as strings) of a mangled or demangled ``mpk::`` kernel."""
    if name.startswith("_ZN3mpk"):
        rest = name[len("_ZN3mpk"):]
        digits = re.match(r"\d+", rest)
        if not digits:
            return name, []
        n = int(digits.group(0))
        base = rest[len(digits.group(0)):len(digits.group(0)) + n]
        rest = rest[len(digits.group(0)) + n:]
        args: List[str] = []
        if rest.startswith("I"):
            pos = 1
            while pos < len(rest):
                m = _MANGLED_ARG.match(rest, pos)
                if not m or m.group(5):
                    break
                args.append(m.group(1) or {"0": "false", "1": "true"}.get(m.group(2) or "", "")
                            or ("_Float16" if m.group(3) else "float"))
                pos = m.end()
        return base, args
    words = name.split("<", 1)[0].split("(", 1)[0].split("::")[-1].split()
    base = words[-1] if words else name
    if "<" not in name:
        return base, []
    inner = name.split("<", 1)[1].rsplit(">", 1)[0]
    return base, [a.strip() for a in inner.split(",")]


def base_kernel_key(name: str) -> str:
    """Kernel role from its name; '@residual' / '@ln' are resolved by ``label_dispatches``."""
    base, args = parse_kernel_name(name)
    if base == "layer_tail_kernel" and len(args) >= 5:
        if args[3] == "false":
            return "layernorm_qkv"
        # layer_tail_kernel<D, F, TM, STAGE1, LAST, QMODE, W, AHD>: AHD > 0 computes attention too
        attn = "attention_" if len(args) >= 8 and args[7] not in ("0", "") else ""
        return attn + ("layer_tail_last" if args[4] == "true" else "layer_tail")
    if base in ("attention32_kernel", "attention_kernel"):
        return "attention"
    if base in ("linear_big_kernel", "linear_kernel"):
        # the epilogue is the integer template argument that follows the input type
        types = [i for i, a in enumerate(args) if a in ("float", "_Float16")]
        index = types[0] + 1 if types else -1
        epi = int(args[index]) if 0 <= index < len(args) and args[index].lstrip("-").isdigit() else -1
        return {0: "qkv_proj", 1: "ffn_in", 2: "@ln", 3: "@residual", 4: "@ln"}.get(epi, "linear")
    if base == "linear_dma_kernel":
        # linear_dma_kernel<EPI, OT>: the epilogue is the first template argument
        epi = int(args[0]) if args and args[0].lstrip("-").isdigit() else -1
        return {0: "qkv_proj", 1: "ffn_in", 3: "@residual"}.get(epi, "linear")
    if base == "linear_xs_kernel":
        # linear_xs_kernel<KS, EPI, OT>: the epilogue is the second template argument
        epi = int(args[1]) if len(args) > 1 and args[1].lstrip("-").isdigit() else -1
        return {0: "qkv_proj", 1: "ffn_in"}.get(epi, "linear")
    if base in ("ffn_ln_kernel", "ffn_wide_kernel", "ffn_roles_kernel"):
        return "ffn_ln"
    if base == "residual_layernorm_kernel":
        return "layernorm"
    if "copyBuffer" in name or "copy_kernel" in name or "elementwise_kernel" in name:
        return "copy"
    return base[:60]


def label_dispatches(names: List[str]) -> List[str]:
    """Per-dispatch kernel keys in launch order.

    The out-projection and the FFN-output projection can be the same kernel
    instantiation; a residual / LayerNorm-epilogue GEMM is the out-projection
    when the last other kernel launched was attention, and the FFN output when
    it was the FFN-in GEMM (in the forward, and in the per-kernel timing loops,
    which launch the kernels in forward order).
    """
    labels = []
    previous = "attention"
    for name in names:
        key = base_kernel_key(name)
        if key.startswith("@"):
            prefix = "ffn_out" if previous == "ffn_in" else "out_proj"
            key = prefix + ("_residual" if key == "@residual" else "_ln")
        else:
            previous = key
        labels.append(key)
    return labels


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


def _csv_rows(path: str):
    import csv
    import glob

    if os.path.isdir(path):
        found = sorted(glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True)
                       or glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True))
        if not found:
            raise FileNotFoundError(f"no rocprofv3 CSV under {path}")
        path = found[0]
    with open(path) as handle:
        return list(csv.DictReader(handle))


def counters_per_dispatch(path: str) -> List[Dict[str, object]]:
    """rocprofv3 counter-collection rows -> one dict per dispatch in dispatch order:
    {"name", "key", "ns", counter: value...}."""
    by_id: Dict[int, Dict[str, object]] = {}
    for row in _csv_rows(path):
        did = int(row["Dispatch_Id"])
        entry = by_id.setdefault(did, {"name": row["Kernel_Name"],
                                       "ns": float(row["End_Timestamp"]) - float(row["Start_Timestamp"])})
        entry[row["Counter_Name"]] = entry.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
    ordered = [by_id[k] for k in sorted(by_id)]
    for entry, key in zip(ordered, label_dispatches([e["name"] for e in ordered])):
        entry["key"] = key
    return ordered


def trace_per_dispatch(path: str) -> List[Dict[str, object]]:
    """rocprofv3 kernel-trace rows -> [{"name", "key", "ns"}] in dispatch order."""
    rows = sorted(_csv_rows(path), key=lambda r: int(r["Dispatch_Id"]))
    out = [{"name": r["Kernel_Name"], "ns": float(r["End_Timestamp"]) - float(r["Start_Timestamp"])} for r in rows]
    for entry, key in zip(out, label_dispatches([e["name"] for e in out])):
        entry["key"] = key
    return out


def _mean_by_key(entries, field: str) -> Dict[str, float]:
    sums: Dict[str, float] = {}
    counts: Dict[str, int] = {}
    for e in entries:
        if field in e:
            sums[e["key"]] = sums.get(e["key"], 0.0) + float(e[field])
            counts[e["key"]] = counts.get(e["key"], 0) + 1
    return {k: sums[k] / counts[k] for k in sums}


def _merge_json(path: str, config_name: str, table: Dict[str, object], extra: Dict[str, object]) -> None:
    import json

    try:
        with open(path) as handle:
            old = json.load(handle)
    except (OSError, ValueError):
        old = {}
    old.update(extra)
    old[config_name] = table
    with open(path, "w") as handle:
        json.dump(old, handle, indent=1, sort_keys=True)


def traffic_summary(fetch_path: str, write_path: str) -> Dict[str, object]:
    """HBM bytes per launch per kernel key from FETCH_SIZE and WRITE_SIZE runs (KiB per dispatch)."""
    fetch = counters_per_dispatch(fetch_path)
    write = counters_per_dispatch(write_path)
    copy_f = max((e["FETCH_SIZE"] for e in fetch if e["key"] == "copy"), default=0.0)
    copy_w = max((e["WRITE_SIZE"] for e in write if e["key"] == "copy"), default=0.0)
    f_scale = CALIBRATION_BYTES / (copy_f * 1024.0) if copy_f else 1.0
    w_scale = CALIBRATION_BYTES / (copy_w * 1024.0) if copy_w else 1.0
    fmean = _mean_by_key([e for e in fetch if e["key"] != "copy"], "FETCH_SIZE")
    wmean = _mean_by_key([e for e in write if e["key"] != "copy"], "WRITE_SIZE")
    table = {}
    for key in sorted(set(fmean) | set(wmean)):
        fb = fmean.get(key, 0.0) * 1024.0 * f_scale
        wb = wmean.get(key, 0.0) * 1024.0 * w_scale
        table[key] = {"fetch_bytes": fb, "write_bytes": wb, "bytes_per_launch": fb + wb}
    calibration = {"copy_bytes": CALIBRATION_BYTES, "fetch_scale": f_scale, "write_scale": w_scale}
    return {"kernels": table, "calibration": calibration}


def mfma_summary(counter_path: str, trace_path: str) -> Dict[str, object]:
    """MFMA busy fraction and counted MFMA FLOPs per kernel key.

    busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / XCDs x SIMDs), the share of
    SIMD cycles with the matrix core busy while the kernel ran;
    counted FLOPs = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512; rate = counted FLOPs / the
    kernel-trace average duration (counter runs serialise and slow dispatches).
    """
    entries = counters_per_dispatch(counter_path)
    durations = _mean_by_key(trace_per_dispatch(trace_path), "ns")
    table = {}
    for key in sorted({e["key"] for e in entries}):
        if key == "copy":
            continue
        sel = [e for e in entries if e["key"] == key]
        busy = [e["SQ_VALU_MFMA_BUSY_CYCLES"] * XCD_PER_GPU / (e["GRBM_GUI_ACTIVE"] * SIMD_PER_GPU)
                for e in sel if e.get("GRBM_GUI_ACTIVE")]
        flops = [e["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512.0 for e in sel if "SQ_INSTS_VALU_MFMA_MOPS_F16" in e]
        row = {
            "dispatches": len(sel),
            "mfma_busy": sum(busy) / len(busy) if busy else None,
            "mfma_flops_per_launch": sum(flops) / len(flops) if flops else None,
            "valu_insts_per_launch": _mean_by_key(sel, "SQ_INSTS_VALU").get(key),
            "mfma_insts_per_launch": _mean_by_key(sel, "SQ_INSTS_MFMA").get(key),
            "trace_avg_us": durations[key] / 1e3 if key in durations else None,
        }
        if row["mfma_flops_per_launch"] and row["trace_avg_us"]:
            row["mfma_tflops"] = row["mfma_flops_per_launch"] / (row["trace_avg_us"] * 1e-6) / 1e12
        table[key] = row
    return table


CONFIG_ORDER = ("cfg1", "cfg2", "cfg3", "cfg4", "cfg5")


def results_table(runs_dir: str, profiles_dir: str) -> str:
    """Markdown results table: bench lines, kernel-trace averages and PMC counters."""
    import json

    def load(path):
        try:
            with open(path) as handle:
                return json.load(handle)
        except (OSError, ValueError):
            return {}

    traffic = load(os.path.join(profiles_dir, "hbm_traffic.json"))
    mfma = load(os.path.join(profiles_dir, "mfma_counters.json"))
    lines = [
        "| cfg | shape (B,S,D,H,F,L) | median ms | tokens/s | fwd floor ms | fwd roofline frac | "
        "max abs err (bench rows) | CPU strict-FP32 tokens/s (threads) | GPU/CPU |",
        "|---|---|---|---|---|---|---|---|---|",
    ]
    kernel_lines = [
        "| cfg | kernel | launches/fwd | bench avg us | rocprof avg us | bound | achieved | frac of peak | "
        "TFLOP/s | GB/s | PMC HBM MB/launch (x algorithmic) | MFMA busy | counted MFMA TFLOP/s |",
        "|---|---|---|---|---|---|---|---|---|---|---|---|---|",
    ]
    for name in CONFIG_ORDER:
        bench = load(os.path.join(runs_dir, f"bench_{name}.json"))
        if not bench:
            continue
        cfg = bench["config"]
        shape = ",".join(str(cfg[k]) for k in ("batch", "seq_len", "d_model", "heads", "ffn_dim", "layers"))
        cpu = bench.get("cpu_baseline") or {}
        par = bench.get("parity") or {}
        ratio = f"{bench['value'] / cpu['value']:.0f}x" if cpu.get("value") else "-"
        lines.append(
            f"| {name} | {shape} | {bench['median_ms']:.4g} | {bench['value']:.4g} | "
            f"{bench['forward_roofline_floor_ms']:.4g} | {bench['forward_roofline_frac']:.3f} | "
            f"{par.get('max_abs', float('nan')):.3g} ({par.get('failed', '?')}/{par.get('elements', '?')} failed) | "
            f"{cpu.get('value', float('nan')):.4g} ({cpu.get('cores', '?')}) | {ratio} |"
        )
        trace_dir = os.path.join(runs_dir, f"prof_{name}")
        try:
            rocprof = _mean_by_key(trace_per_dispatch(trace_dir), "ns")
        except (OSError, FileNotFoundError):
            rocprof = {}
        tcfg = (traffic.get(name) or {})
        tcfg = tcfg.get("kernels", tcfg)
        mcfg = mfma.get(name) or {}
        for k in bench["kernels"]:
            key = k["kernel"]
            rp = f"{rocprof[key] / 1e3:.1f}" if key in rocprof else "-"
            tr = tcfg.get(key)
            alg = k.get("bytes") or k.get("algorithmic_bytes")
            if tr:
                ratio_t = f" ({tr['bytes_per_launch'] / alg:.2f}x)" if alg else ""
                tr_s = f"{tr['bytes_per_launch'] / 1e6:.1f}{ratio_t}"
            else:
                tr_s = "-"
            mc = mcfg.get(key) or {}
            busy = f"{mc['mfma_busy']:.3f}" if mc.get("mfma_busy") is not None else "-"
            ctf = f"{mc['mfma_tflops']:.0f}" if mc.get("mfma_tflops") else "-"
            kernel_lines.append(
                f"| {name} | {key} | {k['launches_per_forward']} | {k['avg_us']:.2f} | {rp} | {k['bound']} | "
                f"{k['achieved']:.4g} {k['unit']} | {k['frac']:.3f} | {k['tflops']:.1f} | {k['gbps']:.0f} | "
                f"{tr_s} | {busy} | {ctf} |"
            )
    return "\n".join(lines) + "\n\n" + "\n".join(kernel_lines) + "\n"


RESULTS_HEADER = """# Forward results on one MI355X: all five benchmark configurations

Regenerate this page (repository root; the GPU-box commands write `gpurun_out/`):

```
# on the GPU box, per configuration N = 1..5
python bench.py --config cfgN --json-out gpurun_out/bench_cfgN.json
cd /tmp && export TMPDIR=/tmp && rocprofv3 --kernel-trace --stats --output-format csv \\
    -d $GRAFT_REPO_ROOT/gpurun_out/prof_cfgN -o run -- \\
    python3 $GRAFT_REPO_ROOT/bench.py --config cfgN --no-cpu-baseline --steps 20 --warmup 3
# on the GPU box, counter passes for N = 1..5 (one rocprofv3 run per pass; eager forward of
# one microbatch, 3 iterations, after a 1 GiB copy that calibrates FETCH_SIZE / WRITE_SIZE)
cd /tmp && export TMPDIR=/tmp && PYTHONPATH=$GRAFT_REPO_ROOT rocprofv3 --pmc FETCH_SIZE --output-format csv \\
    -d $GRAFT_REPO_ROOT/gpurun_out/pmc_cfgN_FETCH_SIZE -o run -- python3 -m tiktoktechjam2026_amd.profiling run --config cfgN
(same with --pmc WRITE_SIZE -> pmc_cfgN_WRITE_SIZE)
(same with --pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU SQ_INSTS_MFMA SQ_WAVES \\
    GRBM_GUI_ACTIVE -> pmc_cfgN_SQ_VALU_MFMA_BUSY_CYCLES)
(same with --kernel-trace instead of --pmc ... -> trace_run_cfgN: the durations the MFMA rates use)
# then, on any host
python -m tiktoktechjam2026_amd.profiling traffic gpurun_out/pmc_cfgN_FETCH_SIZE gpurun_out/pmc_cfgN_WRITE_SIZE --config cfgN
python -m tiktoktechjam2026_amd.profiling mfma gpurun_out/pmc_cfgN_SQ_VALU_MFMA_BUSY_CYCLES gpurun_out/trace_run_cfgN --config cfgN
python -m tiktoktechjam2026_amd.profiling table gpurun_out --out profiles/forward_all_configs_mi355x.md
```

- median ms: HIP-event median per forward (HIP-graph replay for cfg1-4; cfg5 runs eagerly as
  8 microbatches of 64 into a preallocated output, and its figures cover all 512 sequences).
- fwd floor: the forward's roofline time, the sum over kernels of max(FLOPs / 2.5 PFLOP/s,
  algorithmic bytes / 8 TB/s); fwd roofline frac = floor / measured ms per step.
- errors: GPU output against the strict-FP32 oracle under |err| <= 0.002 or <= 0.02 |ref| on the
  batch rows the CPU baseline computes; every element of every configuration is compared in
  `parity_all_configs_mi355x.md`.
- CPU: the strict-FP32 oracle on the box's host CPU (threads = the process's CPU affinity), a
  bounded sample of whole sequences of the same input.
- PMC HBM bytes: FETCH_SIZE + WRITE_SIZE per dispatch (KiB), scaled by what the same counters read
  for the 1 GiB copy kernel (`calibration` in `hbm_traffic.json`), against the algorithmic bytes.
- MFMA busy: SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs); counted MFMA
  TFLOP/s: SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 FLOPs / the kernel-trace duration (the kernels also
  run MFMAs that the algorithmic count does not include, such as attention's row sums and the
  full blocks on the causal diagonal).

"""


def results_page(runs_dir: str, profiles_dir: str) -> str:
    return RESULTS_HEADER + results_table(runs_dir, profiles_dir)


def trace_page(prof_dir: str, config_name: str) -> str:
    """Markdown summary of a rocprofv3 ``--kernel-trace --stats`` run of bench.py."""
    import csv
    import glob

    found = sorted(glob.glob(os.path.join(prof_dir, "**", "*kernel_stats.csv"), recursive=True))
    if not found:
        raise FileNotFoundError(f"no kernel_stats.csv under {prof_dir}")
    with open(found[0]) as handle:
        rows = list(csv.DictReader(handle))
    from .config import BENCHMARK_CONFIGS

    c = BENCHMARK_CONFIGS[config_name]
    lines = [
        f"# rocprofv3 kernel trace: {config_name} forward (B{c.batch_size} S{c.seq_len} D{c.d_model} "
        f"H{c.num_heads} F{c.ffn_dim} L{c.num_layers})",
        "",
        "Command (repository root on the GPU box), then the summary on any host:",
        "",
        "```",
        "cd /tmp && export TMPDIR=/tmp && rocprofv3 --kernel-trace --stats --output-format csv \\",
        f"    -d $GRAFT_REPO_ROOT/gpurun_out/prof_{config_name} -o run -- \\",
        f"    python3 $GRAFT_REPO_ROOT/bench.py --config {config_name} --no-cpu-baseline --steps 20 --warmup 3",
        f"python -m tiktoktechjam2026_amd.profiling trace-page gpurun_out/prof_{config_name} --config {config_name} "
        f"--out profiles/{config_name}_forward_kernel_trace.md",
        "```",
        "",
        "The run covers bench.py's warm-up and timed forwards plus its per-kernel timing loops, so",
        "call counts exceed the launches of one forward.",
        "",
        "| kernel | role | calls | avg us | min us | max us | share of GPU time |",
        "|---|---|---|---|---|---|---|",
    ]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        name = r["Name"]
        base, args = parse_kernel_name(name)
        role = base_kernel_key(name)
        role = {"@residual": "residual GEMM", "@ln": "LayerNorm-epilogue GEMM"}.get(role, role)
        own = name.startswith("_ZN3mpk") or "mpk::" in name
        label = f"`{base}<{', '.join(args)}>`" if args and own else f"`{base}`"
        lines.append(
            f"| {label} | {role} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
            f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.1f} % |"
        )
    return "\n".join(lines) + "\n"


def parity_table(records_path: str, commit: Optional[str] = None) -> str:
    import json

    with open(records_path) as handle:
        records = json.load(handle)
    order = {n: i for i, n in enumerate(CONFIG_ORDER)}
    records.sort(key=lambda r: (order.get(r["config"], 99), r["trial"]))
    lines = [
        "# Whole-output parity on one MI355X: all five benchmark configurations, three seeds",
        "",
        "Every output element of the HIP forward against the strict-FP32 oracle (run on the GPU with TF32",
        "off; one batch row per configuration also through the CPU oracle, last column) under the",
        "reference's rule |err| <= 0.002 or |err| <= 0.02 |ref|, both finite. cfg5 runs all 512",
        "sequences as eight microbatches of 64 through `PreallocatedMicrobatchModel`.",
        "",
        "```",
        "# on the GPU box (repository root)",
        "MPK_PARITY_JSON=gpurun_out/parity_full.json python -u -m pytest tests/test_parity_full_gpu.py -m gpu -s -q",
        "python -m tiktoktechjam2026_amd.profiling parity-table gpurun_out/parity_full.json "
        "--out profiles/parity_all_configs_mi355x.md",
        "```",
        "",
    ]
    if commit:
        lines += [f"Kernels as of commit `{commit}`.", ""]
    lines += [
        "| cfg | trial | input seed | elements compared | failed | max abs err | max rel err | mean abs err | "
        "GPU vs CPU oracle (one row) |",
        "|---|---|---|---|---|---|---|---|---|",
    ]
    for r in records:
        cross = r.get("gpu_vs_cpu_oracle_max_abs")
        lines.append(
            f"| {r['config']} | {r['trial']} | {r['input_seed']} | {r['elements']:,} | {r['failed']} | "
            f"{r['max_abs']:.6g} | {r['max_rel']:.6g} | {r['mean_abs']:.3g} | "
            f"{'-' if cross is None else f'{cross:.2g}'} |"
        )
    return "\n".join(lines) + "\n"


def _main(argv=None) -> None:
    import argparse

    parser = argparse.ArgumentParser(prog="python -m tiktoktechjam2026_amd.profiling")
    sub = parser.add_subparsers(dest="cmd", required=True)
    p_run = sub.add_parser("run")
    p_run.add_argument("--config", default="cfg5")
    p_run.add_argument("--iters", type=int, default=3)
    p_tr = sub.add_parser("traffic")
    p_tr.add_argument("fetch")
    p_tr.add_argument("write")
    p_tr.add_argument("--config", required=True)
    p_tr.add_argument("--out", default="profiles/hbm_traffic.json")
    p_mf = sub.add_parser("mfma")
    p_mf.add_argument("counters")
    p_mf.add_argument("trace")
    p_mf.add_argument("--config", required=True)
    p_mf.add_argument("--out", default="profiles/mfma_counters.json")
    p_tab = sub.add_parser("table")
    p_tab.add_argument("runs_dir")
    p_tab.add_argument("--profiles", default="profiles")
    p_tab.add_argument("--out", default=None)
    p_tp = sub.add_parser("trace-page")
    p_tp.add_argument("prof_dir")
    p_tp.add_argument("--config", required=True)
    p_tp.add_argument("--out", default=None)
    p_par = sub.add_parser("parity-table")
    p_par.add_argument("records")
    p_par.add_argument("--commit", default=None)
    p_par.add_argument("--out", default=None)
    args = parser.parse_args(argv)
    if args.cmd == "run":
        _run(args.config, args.iters)
    elif args.cmd == "traffic":
        summary = traffic_summary(args.fetch, args.write)
        _merge_json(args.out, args.config, summary["kernels"], {"calibration": summary["calibration"]})
        print(summary)
    elif args.cmd == "mfma":
        table = mfma_summary(args.counters, args.trace)
        _merge_json(args.out, args.config, table, {"simd_per_gpu": SIMD_PER_GPU, "xcd_per_gpu": XCD_PER_GPU})
        print(table)
    else:
        if args.cmd == "table":
            text = results_page(args.runs_dir, args.profiles)
        elif args.cmd == "trace-page":
            text = trace_page(args.prof_dir, args.config)
        else:
            text = parity_table(args.records, args.commit)
        if args.out:
            with open(args.out, "w") as handle:
                handle.write(text)
        print(text, end="")


if __name__ == "__main__":
    _main()
