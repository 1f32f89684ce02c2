"""Build recipe for ``libnanokv.so``: the HIP kernels plus the C ABI declared
in ``include/nanokv.h``, compiled with hipcc for gfx950 into this package
directory (in-tree, so the library travels with the source tree).

Run ``python -m nanokv.build`` (with ``nano-vllm-multimodal_amd`` on
``sys.path``) or call :func:`build`.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR.parent / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parents[1] / "include"
LIBRARY_PATH = PACKAGE_DIR / "libnanokv.so"
SOURCES = (
    "nkv_api.hip",
    "nkv_store.hip",
    "nkv_gather.hip",
    "nkv_pack.hip",
    "nkv_transfer.hip",
    "nkv_attention.hip",
    "nkv_prefill.hip",
    "nkv_pool.hip",
    "nkv_noalloc.hip",
    "nkv_store_gather.hip",
)
OFFLOAD_ARCH = "gfx950"
HIPCC_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    # Packed FP32 instructions are kept out of every code object.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


# Headers the sources include: part of the fingerprint with the sources.
HEADERS = ("nkv_common.h", "nkv_mfma.h")


def fingerprint_files(source_dir: Path = SOURCE_DIR, include_dir: Path = INCLUDE_DIR) -> list[Path]:
    return ([source_dir / name for name in SOURCES] + [source_dir / name for name in HEADERS]
            + [include_dir / "nanokv.h"])


def source_fingerprint(source_dir: Path = SOURCE_DIR, include_dir: Path = INCLUDE_DIR) -> str:
    """16 hex digits of a SHA-256 over every source and header (name and
    bytes), the compiler flags and the offload architecture, each field
    length-prefixed so that no two inputs collide by concatenation.  The
    reference names its extension build after the same kind of digest
    (nanovllm/layers/paged_kv/loader.py:47-85)."""
    digest = hashlib.sha256()
    fields: list[bytes] = []
    for path in fingerprint_files(Path(source_dir), Path(include_dir)):
        fields += [path.name.encode(), path.read_bytes()]
    fields += ["\0".join(HIPCC_FLAGS).encode(), OFFLOAD_ARCH.encode()]
    for field in fields:
        digest.update(len(field).to_bytes(8, "little"))
        digest.update(field)
    return digest.hexdigest()[:16]


def config_tag(defines: dict[str, object] | None = None) -> str:
    """"default", or 8 hex digits of the launch-shape defines."""
    if not defines:
        return "default"
    text = "\0".join(f"{key}={value}" for key, value in sorted(defines.items()))
    return hashlib.sha256(text.encode()).hexdigest()[:8]


def build_id(defines: dict[str, object] | None = None, source_dir: Path = SOURCE_DIR,
             include_dir: Path = INCLUDE_DIR) -> str:
    """The id nkv_build_id() of a library built from these files returns."""
    return f"{source_fingerprint(source_dir, include_dir)}-{config_tag(defines)}"


def hipcc_path() -> str:
    candidates = []
    rocm = os.environ.get("ROCM_PATH") or os.environ.get("HIP_PATH")
    if rocm:
        candidates.append(Path(rocm) / "bin" / "hipcc")
    candidates.append(Path("/opt/rocm/bin/hipcc"))
    for candidate in candidates:
        if candidate.is_file() and os.access(candidate, os.X_OK):
            return str(candidate)
    found = shutil.which("hipcc")
    if found:
        return found
    raise RuntimeError("hipcc not found (set ROCM_PATH); cannot build libnanokv.so")


def build_command(output: Path, defines: dict[str, object] | None = None,
                  source_dir: Path = SOURCE_DIR, include_dir: Path = INCLUDE_DIR) -> list[str]:
    identity = build_id(defines, source_dir, include_dir)
    return [
        hipcc_path(),
        *HIPCC_FLAGS,
        *(f"-D{key}={value}" for key, value in (defines or {}).items()),
        f'-DNKV_BUILD_ID="{identity}"',
        f"-I{include_dir}",
        *(str(Path(source_dir) / name) for name in SOURCES),
        "-o",
        str(output),
    ]


def build(*, verbose: bool = False, output: Path | None = None,
          defines: dict[str, object] | None = None, source_dir: Path | None = None,
          include_dir: Path | None = None) -> Path:
    """Compile the library (always, even if a build exists) and install it
    atomically at ``output`` (default :data:`LIBRARY_PATH`).  ``defines``
    override the kernels' compile-time launch-shape knobs
    (NKV_GATHER_THREADS, NKV_GATHER_UNROLL, NKV_GATHER_NT_LOADS,
    NKV_GATHER_NT_STORES, NKV_GATHER_CHUNK_BYTES).  The library reports
    :func:`build_id` of its sources and defines through nkv_build_id()."""
    target = Path(output) if output is not None else LIBRARY_PATH
    source_dir = Path(source_dir) if source_dir is not None else SOURCE_DIR
    include_dir = Path(include_dir) if include_dir is not None else INCLUDE_DIR
    missing = [str(path) for path in fingerprint_files(source_dir, include_dir) if not path.is_file()]
    if missing:
        raise RuntimeError(f"nanokv sources missing: {', '.join(missing)}")
    with tempfile.TemporaryDirectory(prefix="nanokv-build-") as tmp:
        output = Path(tmp) / LIBRARY_PATH.name
        command = build_command(output, defines, source_dir, include_dir)
        if verbose:
            print(" ".join(command), flush=True)
        result = subprocess.run(command, capture_output=True, text=True)
        diagnostics = "\n".join(
            line
            for line in (result.stdout + result.stderr).splitlines()
            # The host pass does not know the GPU target feature; harmless.
            if "packed-fp32-ops" not in line
        ).strip()
        if result.returncode != 0:
            raise RuntimeError(
                f"hipcc failed ({result.returncode}) building libnanokv.so:\n{diagnostics}"
            )
        if diagnostics and verbose:
            print(diagnostics, flush=True)
        target.parent.mkdir(parents=True, exist_ok=True)
        staged = target.with_name(target.name + ".tmp")
        shutil.copyfile(output, staged)
        os.replace(staged, target)
    return target


# ------------------------------------------------------------ host binding
#
# _nkv_host: the backend's per-call store / gather path in C++ (csrc/
# nkv_host.cpp), a CPython extension compiled with g++ against torch's
# headers (it has no device code).  It is bound to the torch it was built
# against, so torch's version is part of its fingerprint.

HOST_SOURCE = "nkv_host.cpp"
HOST_FLAGS = ("-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wno-unused-function")


def host_module_path() -> Path:
    import sysconfig

    return PACKAGE_DIR / f"_nkv_host{sysconfig.get_config_var('EXT_SUFFIX')}"


def host_build_id(source_dir: Path = SOURCE_DIR, include_dir: Path = INCLUDE_DIR) -> str:
    """16 hex digits of a SHA-256 over the binding's source, the C ABI
    header, its flags and the torch version it compiles against."""
    import torch

    digest = hashlib.sha256()
    fields = [HOST_SOURCE.encode(), (Path(source_dir) / HOST_SOURCE).read_bytes(),
              (Path(include_dir) / "nanokv.h").read_bytes(), "\0".join(HOST_FLAGS).encode(),
              torch.__version__.encode(), str(torch._C._GLIBCXX_USE_CXX11_ABI).encode()]
    for field in fields:
        digest.update(len(field).to_bytes(8, "little"))
        digest.update(field)
    return digest.hexdigest()[:16]


def host_build_command(output: Path, source_dir: Path = SOURCE_DIR,
                       include_dir: Path = INCLUDE_DIR) -> list[str]:
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    compiler = shutil.which("g++") or "g++"
    includes = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(include_dir)]
    libraries = cpp_extension.library_paths()
    return [
        compiler, *HOST_FLAGS,
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
        "-DTORCH_EXTENSION_NAME=_nkv_host", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f'-DNKV_HOST_BUILD_ID="{host_build_id(source_dir, include_dir)}"',
        *(f"-I{path}" for path in includes),
        str(Path(source_dir) / HOST_SOURCE), "-o", str(output),
        *(f"-L{path}" for path in libraries), *(f"-Wl,-rpath,{path}" for path in libraries),
        "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
    ]


def build_host(*, verbose: bool = False, output: Path | None = None,
               source_dir: Path | None = None, include_dir: Path | None = None) -> Path:
    """Compile the host binding (always) and install it atomically at
    ``output`` (default :func:`host_module_path`)."""
    target = Path(output) if output is not None else host_module_path()
    source_dir = Path(source_dir) if source_dir is not None else SOURCE_DIR
    include_dir = Path(include_dir) if include_dir is not None else INCLUDE_DIR
    with tempfile.TemporaryDirectory(prefix="nanokv-host-") as tmp:
        staged_build = Path(tmp) / target.name
        command = host_build_command(staged_build, source_dir, include_dir)
        if verbose:
            print(" ".join(command), flush=True)
        result = subprocess.run(command, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"g++ failed ({result.returncode}) building {target.name}:\n"
                               f"{(result.stdout + result.stderr).strip()}")
        target.parent.mkdir(parents=True, exist_ok=True)
        staged = target.with_name(target.name + ".tmp")
        shutil.copyfile(staged_build, staged)
        os.replace(staged, target)
    return target


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
    print(build_host(verbose="-v" in sys.argv))
