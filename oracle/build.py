"""Build the CPU oracle ``oracle/liblct_oracle.so`` with gcc (+OpenMP).

TEST INFRASTRUCTURE: the oracle is the parity checker and the host-core
baseline; the product library never links it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SOURCE = ORACLE_DIR / "lct_oracle.c"
LIBRARY = ORACLE_DIR / "liblct_oracle.so"


def build_oracle() -> Path:
    """Compile the oracle; always rebuilds.  Returns the library path."""
    cc = os.environ.get("CC") or shutil.which("gcc") or "cc"
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [cc, "-O3", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-Wall", "-Wextra",
           str(SOURCE), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"oracle build failed: {' '.join(cmd)}\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build_oracle())
