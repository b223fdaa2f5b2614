"""Builds libdllm_hip.so (the gfx950 HIP kernels behind include/dllm_hip.h) in-tree with hipcc.

Every translation unit is compiled with -ffp-contract=off (no multiply-add is fused behind the code's back: the only
fused operations are the explicit fma calls on exact float products) and without fast-math, so each + - * / and
sqrt rounds once, as in the reference CPU kernels. Packed FP32 instructions are disabled for all device code.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libdllm_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core accumulators in architectural VGPRs (no AGPR copies around each MFMA)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _compile(source: Path) -> Path:
    obj = BUILD / (source.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr[-4000:]}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objects = list(pool.map(_compile, sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr[-4000:]}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


def build_oracle() -> None:
    """The CPU checker (oracle/liboracle.so) and, where the reference checkout exists, oracle/_ref."""
    subprocess.run(["make", "-C", str(ROOT / "oracle")], check=True, capture_output=True)


if __name__ == "__main__":
    build(verbose=True)
    build_oracle()
