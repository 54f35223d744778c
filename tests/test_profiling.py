"""CPU tests of the rocprofv3 summary helpers: kernel-name parsing, per-dispatch labelling of the
projection roles, and the counter arithmetic on hand-made CSV files."""

from __future__ import annotations

import csv
import json

import pytest

from tiktoktechjam2026_amd import profiling

BIG_LN = "_ZN3mpk17linear_big_kernelILi256ELi2EDF16_Li4EDF16_EEvNS_10LinearArgsE"
BIG_RES = "_ZN3mpk17linear_big_kernelILi256ELi2EDF16_Li3EfEEvNS_10LinearArgsE"
BIG_QKV = "_ZN3mpk17linear_big_kernelILi256ELi2EfLi0EDF16_EEvNS_10LinearArgsE"
BIG_GELU = "_ZN3mpk17linear_big_kernelILi256ELi2EDF16_Li1EDF16_EEvNS_10LinearArgsE"
ATTN = "_ZN3mpk18attention32_kernelILi32ELi8ELi64EDF16_DF16_Lb0EEEvNS_8AttnArgsE"
TAIL = "_ZN3mpk17layer_tail_kernelILi128ELi128ELi1ELb1ELb0ELi1EEEvNS_8TailArgsE"
TAIL_LAST = "_ZN3mpk17layer_tail_kernelILi128ELi128ELi1ELb1ELb1ELi1EEEvNS_8TailArgsE"
HEAD = "_ZN3mpk17layer_tail_kernelILi128ELi32ELi1ELb0ELb0ELi1EEEvNS_8TailArgsE"
COPY = "__amd_rocclr_copyBuffer"


# the current template layout <BM, BN, BK, STAGES, XT, EPI, OT> and the role-split FFN
BIG_LN_512 = "_ZN3mpk17linear_big_kernelILi128ELi512ELi32ELi2EDF16_Li4EDF16_EEvNS_10LinearArgsE"
BIG_QKV_256 = "_ZN3mpk17linear_big_kernelILi256ELi256ELi64ELi2EDF16_Li0EDF16_EEvNS_10LinearArgsE"
FFN_ROLES = "_ZN3mpk16ffn_roles_kernelILi256EDF16_DF16_EEvNS_7FfnArgsE"


def test_roles_of_current_kernel_templates():
    assert profiling.parse_kernel_name(BIG_LN_512) == (
        "linear_big_kernel", ["128", "512", "32", "2", "_Float16", "4", "_Float16"])
    assert [profiling.base_kernel_key(n) for n in (BIG_LN_512, BIG_QKV_256, FFN_ROLES)] == ["@ln", "qkv_proj", "ffn_ln"]
    dma = ["_ZN3mpk17linear_dma_kernelILi0EDF16_EEvNS_10LinearArgsE", "_ZN3mpk17linear_dma_kernelILi1EDF16_EEvNS_10LinearArgsE",
           "_ZN3mpk17linear_dma_kernelILi3EfEEvNS_10LinearArgsE"]
    assert profiling.parse_kernel_name(dma[2]) == ("linear_dma_kernel", ["3", "float"])
    assert [profiling.base_kernel_key(n) for n in dma] == ["qkv_proj", "ffn_in", "@residual"]
    xs = ["_ZN3mpk16linear_xs_kernelILi8ELi0EDF16_EEvNS_10LinearArgsE", "_ZN3mpk16linear_xs_kernelILi4ELi1EfEEvNS_10LinearArgsE"]
    assert profiling.parse_kernel_name(xs[1]) == ("linear_xs_kernel", ["4", "1", "float"])
    assert [profiling.base_kernel_key(n) for n in xs] == ["qkv_proj", "ffn_in"]


def test_parse_mangled_and_demangled_names():
    assert profiling.parse_kernel_name(BIG_LN) == ("linear_big_kernel", ["256", "2", "_Float16", "4", "_Float16"])
    assert profiling.parse_kernel_name(ATTN)[1][-1] == "false"
    assert profiling.parse_kernel_name("void mpk::linear_big_kernel<256, 2, float, 0, _Float16>(mpk::LinearArgs)") == (
        "linear_big_kernel", ["256", "2", "float", "0", "_Float16"])
    keys = [profiling.base_kernel_key(n) for n in (BIG_QKV, BIG_GELU, BIG_RES, BIG_LN, ATTN, TAIL, TAIL_LAST, HEAD)]
    assert keys == ["qkv_proj", "ffn_in", "@residual", "@ln", "attention", "layer_tail", "layer_tail_last",
                    "layernorm_qkv"]


def test_label_dispatches_separates_out_projection_from_ffn_output():
    forward = [BIG_QKV, ATTN, BIG_LN, BIG_GELU, BIG_LN] * 2
    assert profiling.label_dispatches(forward) == ["qkv_proj", "attention", "out_proj_ln", "ffn_in", "ffn_out_ln"] * 2
    # per-kernel timing loops: each kernel repeated, in forward order
    loops = [ATTN] * 3 + [BIG_RES] * 3 + [BIG_GELU] * 3 + [BIG_RES] * 3
    assert profiling.label_dispatches(loops)[3:6] == ["out_proj_residual"] * 3
    assert profiling.label_dispatches(loops)[9:] == ["ffn_out_residual"] * 3


def _write_counters(path, dispatches):
    fields = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    with open(path, "w", newline="") as handle:
        writer = csv.DictWriter(handle, fieldnames=fields)
        writer.writeheader()
        for i, (name, counters, ns) in enumerate(dispatches, start=1):
            for counter, value in counters.items():
                writer.writerow({"Dispatch_Id": i, "Kernel_Name": name, "Counter_Name": counter,
                                 "Counter_Value": value, "Start_Timestamp": 1000, "End_Timestamp": 1000 + ns})


def test_traffic_summary_scales_by_the_calibration_copy(tmp_path):
    gib_kib = (1 << 30) / 1024
    fetch = tmp_path / "fetch.csv"
    write = tmp_path / "write.csv"
    # FETCH_SIZE reads half of the copy's bytes, WRITE_SIZE all of them
    _write_counters(fetch, [(COPY, {"FETCH_SIZE": gib_kib / 2}, 10), (ATTN, {"FETCH_SIZE": 1000.0}, 10),
                            (ATTN, {"FETCH_SIZE": 3000.0}, 10)])
    _write_counters(write, [(COPY, {"WRITE_SIZE": gib_kib}, 10), (ATTN, {"WRITE_SIZE": 500.0}, 10),
                            (ATTN, {"WRITE_SIZE": 500.0}, 10)])
    summary = profiling.traffic_summary(str(fetch), str(write))
    assert summary["calibration"]["fetch_scale"] == pytest.approx(2.0)
    row = summary["kernels"]["attention"]
    assert row["fetch_bytes"] == pytest.approx(2000.0 * 1024 * 2.0)
    assert row["write_bytes"] == pytest.approx(500.0 * 1024)
    assert "copy" not in summary["kernels"]


def test_mfma_summary_busy_fraction_and_rate(tmp_path):
    counters = tmp_path / "mfma.csv"
    trace = tmp_path / "trace.csv"
    # GRBM_GUI_ACTIVE arrives summed over the 8 XCDs: 8000 = 1000 cycles of kernel time
    _write_counters(counters, [(ATTN, {"SQ_VALU_MFMA_BUSY_CYCLES": 512.0 * 1000, "GRBM_GUI_ACTIVE": 8000.0,
                                       "SQ_INSTS_VALU_MFMA_MOPS_F16": 1e6}, 5000)])
    with open(trace, "w", newline="") as handle:
        writer = csv.DictWriter(handle, fieldnames=["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        writer.writeheader()
        writer.writerow({"Dispatch_Id": 1, "Kernel_Name": ATTN, "Start_Timestamp": 0, "End_Timestamp": 2000})
    row = profiling.mfma_summary(str(counters), str(trace))["attention"]
    assert row["mfma_busy"] == pytest.approx(0.5)  # 512k busy SIMD-cycles over 1000 cycles x 1024 SIMDs
    assert row["mfma_flops_per_launch"] == pytest.approx(512e6)
    assert row["mfma_tflops"] == pytest.approx(512e6 / 2e-6 / 1e12)


def test_parity_table_orders_records(tmp_path):
    records = [
        {"config": "cfg5", "trial": 0, "input_seed": 1234, "elements": 10, "failed": 0, "max_abs": 1e-3,
         "max_rel": 0.01, "mean_abs": 1e-4, "gpu_vs_cpu_oracle_max_abs": 1e-6},
        {"config": "cfg1", "trial": 1, "input_seed": 1235, "elements": 10, "failed": 0, "max_abs": 1e-3,
         "max_rel": 0.01, "mean_abs": 1e-4, "gpu_vs_cpu_oracle_max_abs": None},
    ]
    path = tmp_path / "records.json"
    path.write_text(json.dumps(records))
    text = profiling.parity_table(str(path), commit="abc1234")
    assert "Kernels as of commit `abc1234`." in text
    rows = [ln for ln in text.splitlines() if ln.startswith("| cfg")][1:]  # after the header row
    assert rows[0].startswith("| cfg1 | 1 |") and rows[1].startswith("| cfg5 | 0 |")


def test_fused_attention_tail_kernels_are_named_and_priced():
    """cfg3 runs attention inside the layer tail: the cost model lists the fused kernels (each
    reading the packed QKV instead of the context) and the trace names map to them."""
    from tiktoktechjam2026_amd import profiling
    from tiktoktechjam2026_amd.config import BENCHMARK_CONFIGS

    cfg3 = BENCHMARK_CONFIGS["cfg3"]
    costs = profiling.forward_costs(cfg3)
    assert set(costs) == {"layernorm_qkv", "attention_layer_tail", "attention_layer_tail_last"}
    m, d = cfg3.batch_size * cfg3.seq_len, cfg3.d_model
    assert costs["attention_layer_tail"].launches_per_forward == cfg3.num_layers - 1
    assert costs["attention_layer_tail"].bytes > m * d * 20 and costs["attention_layer_tail_last"].bytes > m * d * 18
    cfg1 = profiling.forward_costs(BENCHMARK_CONFIGS["cfg1"])  # two-kernel route
    assert "attention" in cfg1 and "layer_tail" in cfg1
    key = profiling.base_kernel_key
    assert key("_ZN3mpk17layer_tail_kernelILi32ELi64ELi1ELb1ELb0ELi1ELi4ELi16EEEvNS_8TailArgsE") == "attention_layer_tail"
    assert key("_ZN3mpk17layer_tail_kernelILi32ELi64ELi1ELb1ELb1ELi1ELi4ELi32EEEvNS_8TailArgsE") == "attention_layer_tail_last"
    assert key("_ZN3mpk17layer_tail_kernelILi128ELi128ELi1ELb1ELb0ELi2ELi4ELi0EEEvNS_8TailArgsE") == "layer_tail"
    assert key("_ZN3mpk17layer_tail_kernelILi128ELi128ELi1ELb0ELb0ELi2ELi4ELi0EEEvNS_8TailArgsE") == "layernorm_qkv"
