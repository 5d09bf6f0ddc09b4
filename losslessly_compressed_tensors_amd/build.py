"""Compile the gfx950 HIP sources into ``lib/liblct_hip.so`` (in-tree).

Usage: ``python -m losslessly_compressed_tensors_amd.build`` or
``build_library()``.  Always recompiles.  Cross-compiles without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "lib"
LIBRARY = LIB_DIR / "liblct_hip.so"
BUILD_DIR = PACKAGE_DIR.parent / "_build" / "lct_hip"

SOURCES = [
    "tables.hip",
    "encode.hip",
    "compress.hip",
    "compaction.hip",
    "tensor_buffer.hip",
    "decode.hip",
    "pointwise.hip",
    "update.hip",
    "noalloc.hip",
    "bandwidth.hip",
]

# Packed FP32 instructions are kept out of the device code: the feature is
# switched off for the device pass (the host pass warns that it does not know
# the feature, which is harmless).
HIPCC_FLAGS = [
    "-O3",
    "--offload-arch=gfx950",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and os.path.exists(candidate):
            return candidate
    raise RuntimeError("hipcc not found (ROCm is required to build liblct_hip.so)")


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"
    text = "\n".join(line for line in (result.stdout + result.stderr).splitlines()
                     if noise not in line and line.strip())
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{text}")
    if text and os.environ.get("LCT_BUILD_VERBOSE"):
        print(text, file=sys.stderr)


def build_library(verbose: bool = False) -> Path:
    """Compile every source and link ``liblct_hip.so``; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    objects = []
    jobs = []
    for name in SOURCES:
        obj = BUILD_DIR / (Path(name).stem + ".o")
        objects.append(str(obj))
        jobs.append([hipcc, *HIPCC_FLAGS, "-c", str(CSRC / name), "-o", str(obj)])
    workers = min(len(jobs), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(_run, jobs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objects, "-o", str(tmp)])
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build_library(verbose=True)
