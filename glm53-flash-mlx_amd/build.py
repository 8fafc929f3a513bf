"""Build libglm53_moe.so (gfx950) in-tree with hipcc.

Every translation unit is compiled for gfx950 only, with packed-FP32 VALU ops
disabled (they are not used by any kernel here and are avoided on purpose),
then linked against the HIP runtime only (no vendor math library).  Objects go to ``_build/`` next to this file; the shared library
is written next to this file so it travels with the source tree.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libglm53_moe.so"
BUILD = PKG / "_build"
SOURCES = ["decode.hip", "step.hip", "grouped.hip", "router.hip", "layout.hip", "synth.hip", "api.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    "-Wall",
    "-Wno-unused-function",
]
# Per-source additions.  grouped.hip: MFMA results in ordinary VGPRs (the
# compiler otherwise parks the chained hi/lo results of the narrow GEMM in
# accumulation registers and copies every element out before folding it).
EXTRA = {"grouped.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: str) -> Path:
    obj = BUILD / (src + ".o")
    cmd = [HIPCC, *COMMON, *EXTRA.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *COMMON, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"hipcc failed on {src}")
    return obj


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError("link of libglm53_moe.so failed")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
