"""Compile the gfx950 HIP sources into the in-tree C-ABI library ``libmpk.so``.

    python -m tiktoktechjam2026_amd.build          # build (always recompiles)

Each ``csrc/*.hip`` file is compiled to an object with ``hipcc
--offload-arch=gfx950`` in parallel, then linked into
``tiktoktechjam2026_amd/libmpk.so`` next to this file, so the library travels
with the source tree.  Packed-FP32 VALU instructions are disabled for all
device code (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from typing import List

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libmpk.so")

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in ordinary VGPRs (no AGPR copies around the
    # VALU epilogues and softmax that consume them)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]


# Per-source additions.  The attention kernel never produces NaN from finite
# inputs (masked scores are -inf, exp2(-inf) = 0), so its max reductions need
# no NaN canonicalisation.
EXTRA_FLAGS = {"attention.hip": ["-fno-honor-nans"]}
# Sources whose kernels keep MFMA accumulators in AGPRs: the wide fused FFN runs one
# wave per SIMD with 32 x D FP32 accumulators, more than the 256 arch VGPRs hold
# beside its operands.
AGPR_ACCUMULATORS = {"ffn_wide.hip"}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP kernels cannot be built")
    return path


def sources() -> List[str]:
    return sorted(os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    name = os.path.basename(src)
    flags = list(COMMON_FLAGS)
    if name in AGPR_ACCUMULATORS:
        i = flags.index("-amdgpu-mfma-vgpr-form")
        del flags[i - 1:i + 1]
    cmd = [_hipcc(), *flags, *EXTRA_FLAGS.get(name, []), "-c", src, "-o", obj]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{proc.stdout}")
    return obj


def build(verbose: bool = True) -> str:
    """Compile every HIP source and link ``libmpk.so``; returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of libmpk.so failed:\n{proc.stdout}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} HIP sources for {ARCH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
