"""Build recipe for the oracle's C restatement (oracle/nkv_oracle.c) with
gcc + OpenMP into oracle/_build/libnkv_oracle.so.

TEST INFRASTRUCTURE ONLY.  The reference's own native path
(csrc/paged_kv/*.cu, *.cpp) needs nvcc, the CUDA runtime and libtorch's CUDA
headers, none of which exist in this image, so there is no oracle/_ref build
of it; the C restatement here is the compiled oracle.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import tempfile
from pathlib import Path

ORACLE_DIR = Path(__file__).resolve().parent
SOURCE = ORACLE_DIR / "nkv_oracle.c"
LIBRARY_PATH = ORACLE_DIR / "_build" / "libnkv_oracle.so"
FLAGS = ("-O2", "-std=c11", "-fPIC", "-shared", "-fopenmp", "-Wall")


def build() -> Path:
    compiler = shutil.which("gcc") or shutil.which("cc")
    if compiler is None:
        raise RuntimeError("no C compiler (gcc) found to build the oracle")
    LIBRARY_PATH.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="nkv-oracle-") as tmp:
        output = Path(tmp) / LIBRARY_PATH.name
        result = subprocess.run(
            [compiler, *FLAGS, str(SOURCE), "-o", str(output)], capture_output=True, text=True
        )
        if result.returncode != 0:
            raise RuntimeError(f"oracle build failed:\n{result.stdout}{result.stderr}")
        staged = LIBRARY_PATH.with_name(LIBRARY_PATH.name + ".tmp")
        shutil.copyfile(output, staged)
        os.replace(staged, LIBRARY_PATH)
    return LIBRARY_PATH


if __name__ == "__main__":
    print(build())
