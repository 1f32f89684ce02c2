"""Build recipe for the C host test of the library's C ABI
(tests/c_host/abi_host.c -> tests/c_host/_build/abi_host).

gcc compiles the C program against include/nanokv.h and the HIP runtime's C
API, and links libnanokv.so (the product) and the oracle's C restatement
(oracle/_build/libnkv_oracle.so, which checks the results) through run paths relative to
the binary, so the built tree runs wherever it is copied.  Both libraries
must be built first (``__graft_entry__.build()`` builds all three in order).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO_ROOT = HERE.parents[1]
SOURCE = HERE / "abi_host.c"
BINARY = HERE / "_build" / "abi_host"
LIBRARY_DIR = REPO_ROOT / "nano-vllm-multimodal_amd" / "nanokv"
ORACLE_DIR = REPO_ROOT / "oracle" / "_build"


def rocm_root() -> Path:
    return Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def build_command(output: Path) -> list[str]:
    rocm = rocm_root()
    relative = lambda target: os.path.relpath(target, BINARY.parent)  # noqa: E731
    return [
        shutil.which("gcc") or "gcc",
        "-O2", "-std=c11", "-Wall", "-Wextra",
        # the HIP runtime's C headers select the AMD platform from this macro
        "-D__HIP_PLATFORM_AMD__",
        f"-I{rocm / 'include'}",
        f"-I{REPO_ROOT / 'include'}",
        str(SOURCE),
        "-o", str(output),
        f"-L{LIBRARY_DIR}", "-l:libnanokv.so",
        f"-L{ORACLE_DIR}", "-l:libnkv_oracle.so",
        f"-L{rocm / 'lib'}", "-lamdhip64",
        f"-Wl,-rpath,$ORIGIN/{relative(LIBRARY_DIR)}",
        f"-Wl,-rpath,$ORIGIN/{relative(ORACLE_DIR)}",
        f"-Wl,-rpath,{rocm / 'lib'}",
    ]


def build() -> Path:
    for needed in (LIBRARY_DIR / "libnanokv.so", ORACLE_DIR / "libnkv_oracle.so"):
        if not needed.is_file():
            raise RuntimeError(f"{needed} is missing: build the library and the oracle first")
    BINARY.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory(prefix="nkv-abi-host-") as tmp:
        output = Path(tmp) / BINARY.name
        result = subprocess.run(build_command(output), capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"C host test build failed:\n{result.stdout}{result.stderr}")
        staged = BINARY.with_name(BINARY.name + ".tmp")
        shutil.copyfile(output, staged)
        os.chmod(staged, 0o755)
        os.replace(staged, BINARY)
    return BINARY


if __name__ == "__main__":
    print(build())
