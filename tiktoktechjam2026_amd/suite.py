"""The reference's 14-case benchmark suite, run through this package's CLI.

Restates ``run_mixed_suite.ps1`` (cases :12-27, per-case flags :31-43, status and
result parsing :44-53, CSV columns :56-62): each case runs
``mixed_precision_benchmark.main`` with the reference's flags (``--causal
--accuracy-trials 1 --warmup 3 --repeats 10 --benchmark-rounds 1``), its
output is kept as ``case_<n>.txt`` and the parsed row goes to ``results.csv``
with the reference's column names.

    cd /path/to/reference && PYTHONPATH=/path/to/this/repo \\
        python -m tiktoktechjam2026_amd.suite --run-id mi355x_suite [--cases 1,7,8] [--out DIR]

The strict-FP32 baseline is the reference's ``torch_transformer_benchmark``
module, imported by the CLI exactly as the reference suite does (so this runs
from the reference checkout, or with ``reference=`` given a module exposing
``BaselineTransformer``).  Differences: cases run in one process (a failing
case is recorded and the suite goes on, as with the reference's per-case
exit codes), and extra CLI flags can be appended to every case.
"""

from __future__ import annotations

import argparse
import contextlib
import csv
import io
import os
import re
import sys
from typing import Dict, Iterable, List, Optional, Sequence

# run_mixed_suite.ps1:12-27 - (case, batch, d_model, heads, seq_len, layers, ffn_dim)
CASES = [
    (1, 64, 128, 4, 128, 4, 128),
    (2, 1, 128, 4, 128, 4, 128),
    (3, 4, 128, 4, 128, 4, 128),
    (4, 16, 128, 4, 128, 4, 128),
    (5, 128, 128, 4, 128, 4, 128),
    (6, 10000, 128, 4, 128, 4, 128),
    (7, 64, 32, 4, 128, 4, 32),
    (8, 64, 1024, 4, 128, 4, 1024),
    (9, 64, 128, 1, 128, 4, 128),
    (10, 64, 128, 2, 128, 4, 128),
    (11, 64, 128, 16, 128, 4, 128),
    (12, 64, 128, 4, 32, 4, 128),
    (13, 64, 128, 4, 1024, 4, 128),
    (14, 32, 1024, 16, 100000, 2, 1024),
]

COLUMNS = [
    "Case", "Batch", "DModel", "Heads", "SeqLen", "Layers", "FfnDim", "Status", "Accuracy", "MaxAbs", "Failed",
    "StrictFp32BaselineMs", "MixedCandidateMs", "Speedup",
]


def case_argv(case: Sequence[int], extra: Iterable[str] = ()) -> List[str]:
    """CLI flags of one suite case (run_mixed_suite.ps1:31-43)."""
    _, batch, d_model, heads, seq_len, layers, ffn = case
    return [
        "--batch-size", str(batch), "--d-model", str(d_model), "--heads", str(heads), "--seq-len", str(seq_len),
        "--ffn-dim", str(ffn), "--layers", str(layers), "--causal", "--accuracy-trials", "1", "--warmup", "3",
        "--repeats", "10", "--benchmark-rounds", "1", *extra,
    ]


def _match(pattern: str, text: str) -> str:
    found = re.search(pattern, text)
    return found.group(1).strip() if found else "N/A"


def parse_case_output(text: str, exit_code: int) -> Dict[str, str]:
    """Status and numbers of one case, by the reference suite's patterns (run_mixed_suite.ps1:44-53)."""
    if exit_code == 0:
        status = "OK"
    elif re.search(r"out of memory|OutOfMemoryError", text):
        status = "OOM"
    else:
        status = "ERROR"
    return {
        "Status": status,
        "Accuracy": _match(r"summary: (PASS|FAIL)", text),
        "MaxAbs": _match(r"summary: (?:PASS|FAIL) \| max_abs=([^|]+)", text),
        "Failed": _match(r"summary: (?:PASS|FAIL).*failed=([^\r\n]+)", text),
        "StrictFp32BaselineMs": _match(r"baseline : median=([0-9.]+) ms", text),
        "MixedCandidateMs": _match(r"optimized: median=([0-9.]+) ms", text),
        "Speedup": _match(r"speedup  : ([0-9.]+)x", text),
    }


def run_case(case: Sequence[int], extra: Iterable[str] = (), reference=None) -> tuple:
    """Run one case in-process; returns (exit_code, captured output)."""
    from . import mixed_precision_benchmark

    buffer = io.StringIO()
    with contextlib.redirect_stdout(buffer), contextlib.redirect_stderr(buffer):
        try:
            code = mixed_precision_benchmark.main(case_argv(case, extra), reference=reference)
        except SystemExit as exc:  # argparse / CLI exits
            code = exc.code if isinstance(exc.code, int) else 1
        except Exception as exc:  # the case fails; the suite goes on (the reference records ERROR/OOM)
            print(f"{type(exc).__name__}: {exc}")
            code = 1
    try:
        import torch

        if torch.cuda.is_available():
            torch.cuda.empty_cache()
    except Exception:
        pass
    return code, buffer.getvalue()


def run_suite(run_id: str, cases: Optional[Sequence[int]] = None, out_dir: Optional[str] = None,
              extra: Iterable[str] = (), reference=None) -> List[Dict[str, str]]:
    folder = out_dir or os.path.join("benchmark_logs", run_id)
    os.makedirs(folder, exist_ok=True)
    selected = [c for c in CASES if cases is None or c[0] in cases]
    rows = []
    for case in selected:
        print(f"CASE {case[0]} START", flush=True)
        code, text = run_case(case, extra, reference)
        with open(os.path.join(folder, f"case_{case[0]}.txt"), "w") as handle:
            handle.write(text)
        parsed = parse_case_output(text, code)
        print(
            f"CASE {case[0]} {parsed['Status']} accuracy={parsed['Accuracy']} "
            f"candidate_ms={parsed['MixedCandidateMs']} speedup={parsed['Speedup']}",
            flush=True,
        )
        row = dict(zip(COLUMNS[:7], (str(v) for v in case)))
        row.update(parsed)
        rows.append(row)
    with open(os.path.join(folder, "results.csv"), "w", newline="") as handle:
        writer = csv.DictWriter(handle, fieldnames=COLUMNS)
        writer.writeheader()
        writer.writerows(rows)
    widths = {c: max(len(c), *(len(r[c]) for r in rows)) if rows else len(c) for c in COLUMNS}
    print(" ".join(c.ljust(widths[c]) for c in COLUMNS))
    for row in rows:
        print(" ".join(row[c].ljust(widths[c]) for c in COLUMNS))
    return rows


def main(argv: Optional[List[str]] = None) -> int:
    parser = argparse.ArgumentParser(description="Run the reference's 14-case suite on the HIP candidate")
    parser.add_argument("--run-id", required=True)
    parser.add_argument("--cases", default=None, help="comma-separated case numbers (default: all 14)")
    parser.add_argument("--out", default=None, help="output folder (default: benchmark_logs/<run-id>)")
    args, extra = parser.parse_known_args(argv)
    cases = [int(c) for c in args.cases.split(",")] if args.cases else None
    run_suite(args.run_id, cases, args.out, extra)
    return 0


if __name__ == "__main__":
    sys.exit(main())
