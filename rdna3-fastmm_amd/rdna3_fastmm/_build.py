"""Compile the gfx950 HIP library ``libfastmm_amd.so`` in-tree.

``python -m rdna3_fastmm._build`` (or ``__graft_entry__.build()``) regenerates
nothing: the per-scheme programs in ``csrc/generated`` are checked in and a
test keeps them equal to the generator's output. Every source is compiled
with ``-ffp-contract=off`` (the transforms must round exactly like the fp32
straight-line programs) and without packed-fp32 instructions.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
import os
from pathlib import Path
import shutil
import subprocess
import sys

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR.parent / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parent.parent / "include"
BUILD_DIR = PACKAGE_DIR.parent / "_build"
LIBRARY_NAME = "libfastmm_amd.so"
LIBRARY_PATH = PACKAGE_DIR / LIBRARY_NAME
ARCH = "gfx950"

SOURCES = ("abi_common.cpp", "transforms.hip", "leaf_gemm.hip")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{SOURCE_DIR}",
    f"-I{INCLUDE_DIR}",
]


def _hipcc() -> str:
    candidate = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(candidate).exists():
        raise RuntimeError("hipcc not found; the fastmm library needs ROCm to build")
    return candidate


def _compile(source: str) -> Path:
    target = BUILD_DIR / (Path(source).stem + ".o")
    language = ["-x", "hip"] if source.endswith(".cpp") else []
    command = [_hipcc(), *COMMON_FLAGS, *language, "-c", str(SOURCE_DIR / source), "-o", str(target)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n{result.stderr}")
    return target


def build_library(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    BUILD_DIR.mkdir(exist_ok=True)
    workers = min(len(SOURCES), max(1, (os.cpu_count() or 2) // 2))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, SOURCES))
    temporary = LIBRARY_PATH.with_suffix(".so.tmp")
    command = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(temporary)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking {LIBRARY_NAME} failed:\n{result.stderr}")
    os.replace(temporary, LIBRARY_PATH)
    if verbose:
        print(f"built {LIBRARY_PATH}")
    return LIBRARY_PATH


if __name__ == "__main__":
    build_library(verbose=True)
    sys.exit(0)
