"""Builds libmlxvs_c.so, the engine's C-ABI library, for gfx950 in-tree.

    python -m mlxvs_amd.build            # compile (always) and link

Every HIP source is compiled by hipcc for --offload-arch=gfx950 with packed
FP32 instructions disabled and floating-point contraction off (so norms and
unit rows round exactly as the CPU restatement in oracle/ does), then linked
into mlxvs_amd/libmlxvs_c.so, exporting only the mlxvs_* C symbols.
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
BUILD = PKG / "_build"
LIB = PKG / "libmlxvs_c.so"

SOURCES = ["knn_float.hip", "knn_hamming.hip", "topk_merge.hip", "scratch.hip", "engine.cpp", "c_api.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _compile(src: str) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    lang = ["-x", "hip"] if src.endswith(".hip") else []
    cmd = [HIPCC, *FLAGS, *lang, "-c", str(CSRC / src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every source and link the library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(len(SOURCES)) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs),
           f"-Wl,--version-script={CSRC / 'exports.map'}", "-Wl,-z,defs", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
