"""ctypes binding of ``libnanokv.so`` (the C ABI of ``include/nanokv.h``).

The library is loaded lazily, once, under a lock (the double-checked load of
the reference's CUDA backend, nanovllm/layers/paged_kv/cuda_backend.py:21-42).
A missing or unloadable library raises ``RuntimeError`` with the path and the
loader's message: there is no fallback path.

A library built from other sources than the ones on disk is refused: the
build bakes a fingerprint of its sources, headers, flags and target into
``nkv_build_id()``, and loading recomputes it from the files (the reference
names its extension build after such a fingerprint and rebuilds when it
changes, nanovllm/layers/paged_kv/loader.py:47-112).  The in-tree library
must match exactly, launch-shape defines included; a ``$NANOKV_LIBRARY``
override (a build with other defines) must match the sources, and its full
id is reported by :func:`build_id`.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from threading import Lock

from nanokv import build as _build
from nanokv.build import LIBRARY_PATH

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p
c_ptr_out = ctypes.POINTER(ctypes.c_void_p)
c_i64_out = ctypes.POINTER(ctypes.c_int64)


class PoolDesc(ctypes.Structure):
    """struct nkv_pool_desc: the device buffer holding a block pool and its
    geometry."""

    _fields_ = [
        ("memory", ctypes.c_void_p),
        ("num_blocks", ctypes.c_int64),
        ("max_seqs", ctypes.c_int64),
        ("max_blocks_per_seq", ctypes.c_int64),
    ]


c_pool = ctypes.POINTER(PoolDesc)

# name -> (restype, argtypes); mirrors include/nanokv.h.
SIGNATURES: dict[str, tuple[object, tuple[object, ...]]] = {
    "nkv_version": (ctypes.c_int, ()),
    "nkv_build_id": (ctypes.c_char_p, ()),
    "nkv_last_error": (ctypes.c_char_p, ()),
    "nkv_store": (
        ctypes.c_int,
        (c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_ptr),
    ),
    "nkv_gather": (
        ctypes.c_int,
        (c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_ptr, c_ptr),
    ),
    "nkv_gather_plan_rows": (c_i64, (c_i64, c_i64, c_i32)),
    "nkv_gather_plan_capacity": (c_i64, (c_i64, c_i64, c_i64, c_i64, c_i32)),
    "nkv_build_gather_plan": (
        ctypes.c_int,
        (c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_ptr, c_i64, c_ptr),
    ),
    "nkv_gather_varlen_planned": (
        ctypes.c_int,
        (c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_ptr, c_ptr, c_ptr),
    ),
    "nkv_gather_varlen": (
        ctypes.c_int,
        (
            c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64,
            c_i32, c_ptr, c_ptr, c_ptr, c_i64, c_ptr,
        ),
    ),
    "nkv_store_gather_plan_bytes": (c_i64, (c_i64, c_i64, c_i64, c_i64, c_i64, c_i32)),
    "nkv_build_store_gather_plan": (
        ctypes.c_int,
        (c_ptr, c_i64, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_ptr, c_i64,
         c_ptr),
    ),
    "nkv_store_gather": (
        ctypes.c_int,
        (c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64,
         c_i64, c_i64, c_i32, c_ptr, c_ptr, c_ptr),
    ),
    "nkv_gather_varlen_noalloc": (
        ctypes.c_int,
        (
            c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64,
            c_i32, c_ptr, c_ptr, c_ptr,
        ),
    ),
    "nkv_pack_decode": (
        ctypes.c_int,
        (c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr),
    ),
    "nkv_pack_prefill": (
        ctypes.c_int,
        (
            c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64,
            c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr,
        ),
    ),
    "nkv_attention_entry_rows": (c_i64, (c_i64,)),
    "nkv_attention_plan_capacity": (c_i64, (c_i64, c_i64, c_i64)),
    "nkv_attention_workspace_bytes": (c_i64, (c_i64, c_i64, c_i64)),
    "nkv_build_attention_plan": (
        ctypes.c_int,
        (c_ptr, c_i64, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr),
    ),
    "nkv_paged_attention_decode": (
        ctypes.c_int,
        (
            c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64, c_ptr, c_i64, c_i64,
            c_i64, c_i64, c_i64, c_i64, ctypes.c_float, c_i32, c_ptr, c_i64, c_ptr, c_i64,
            c_ptr,
        ),
    ),
    "nkv_prefill_tile_tokens": (c_i64, (c_i64,)),
    "nkv_prefill_plan_capacity": (c_i64, (c_i64, c_i64, c_i64)),
    "nkv_build_prefill_plan": (ctypes.c_int, (c_ptr, c_ptr, c_i64, c_i64, c_ptr, c_i64, c_ptr)),
    "nkv_paged_attention_prefill": (
        ctypes.c_int,
        (
            c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_ptr, c_ptr, c_i64, c_i64,
            c_i64, c_i64, c_i64, c_i64, c_i64, ctypes.c_float, c_i32, c_ptr, c_i64, c_ptr,
        ),
    ),
    "nkv_transfer_create": (ctypes.c_int, (c_i32, c_ptr_out)),
    "nkv_transfer_destroy": (ctypes.c_int, (c_ptr,)),
    "nkv_transfer_h2d": (ctypes.c_int, (c_ptr, c_ptr, c_ptr, c_i64, c_ptr, c_i64_out)),
    "nkv_transfer_poll": (ctypes.c_int, (c_ptr, c_i64_out, c_i64_out)),
    "nkv_transfer_synchronize": (ctypes.c_int, (c_ptr,)),
    "nkv_pool_bytes": (c_i64, (c_i64, c_i64, c_i64)),
    "nkv_pool_offsets": (ctypes.c_int, (c_i64, c_i64, c_i64, c_i64_out)),
    "nkv_pool_init": (ctypes.c_int, (c_pool, c_ptr)),
    "nkv_pool_apply": (ctypes.c_int, (c_pool, c_ptr, c_i64, c_ptr, c_i64, c_ptr)),
    "nkv_pack_decode_pool": (
        ctypes.c_int,
        (c_pool, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr, c_ptr,
         c_ptr),
    ),
    "nkv_pack_prefill_pool": (
        ctypes.c_int,
        (c_pool, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_i64, c_i64, c_i64, c_ptr, c_ptr, c_ptr,
         c_ptr, c_ptr, c_ptr, c_ptr, c_ptr),
    ),
}

NKV_POOL_OP_ALLOCATE = 1
NKV_POOL_OP_DEALLOCATE = 2
NKV_POOL_OP_APPEND = 3
NKV_POOL_OP_FENCE = 4
NKV_POOL_ERRORS = {
    1: "unknown op type",
    2: "slot outside [0, max_seqs)",
    3: "allocate on a slot that holds blocks",
    4: "append past max_blocks_per_seq",
    5: "not enough free blocks",
    6: "block id out of range or not owned",
    7: "bad counts or args offset",
}

NKV_DTYPE_FLOAT16 = 0
NKV_DTYPE_BFLOAT16 = 1
NKV_DTYPE_FLOAT32 = 2
NKV_MAX_PLAN_SEQS = 8192
NKV_MAX_PACK_SEQS = 4096
NKV_SCRATCH_BYTES = 4 << 20

_LOCK = Lock()
_LIBRARY: ctypes.CDLL | None = None


def library_path() -> str:
    """The in-tree build, unless NANOKV_LIBRARY names another build of the
    same ABI (e.g. one compiled with different launch-shape knobs)."""
    return os.environ.get("NANOKV_LIBRARY") or str(LIBRARY_PATH)


def verify_build_id(found: str, path: Path, *, override: bool, source_dir: Path = _build.SOURCE_DIR,
                    include_dir: Path = _build.INCLUDE_DIR) -> None:
    """Raise RuntimeError when the library at ``path`` (whose nkv_build_id()
    is ``found``) was not built from the sources in ``source_dir`` and
    ``include_dir``.  Without the sources (an install that ships only the
    library) there is nothing to compare against."""
    if not all(f.is_file() for f in _build.fingerprint_files(Path(source_dir), Path(include_dir))):
        return
    sources = _build.source_fingerprint(source_dir, include_dir)
    expected = f"{sources}-{_build.config_tag(None)}"
    stale = not found.startswith(sources + "-") if override else found != expected
    if stale:
        raise RuntimeError(
            f"{path} is stale: built as {found!r}, the sources in {source_dir} give "
            f"{expected!r}{' (any launch-shape config)' if override else ''}; rebuild it "
            "(__graft_entry__.build() or python -m nanokv.build)")


def open_library(path: Path, *, override: bool = False, source_dir: Path = _build.SOURCE_DIR,
                 include_dir: Path = _build.INCLUDE_DIR) -> ctypes.CDLL:
    """Load the library at ``path``, check its build id against the sources
    and bind every entry point of the ABI."""
    path = Path(path)
    if not path.is_file():
        raise RuntimeError(
            f"nanokv HIP library not built: {path} is missing "
            "(run __graft_entry__.build() or python -m nanokv.build)"
        )
    try:
        library = ctypes.CDLL(str(path))
    except OSError as exc:
        raise RuntimeError(f"failed to load {path}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        try:
            function = getattr(library, name)
        except AttributeError as exc:
            raise RuntimeError(f"{path} does not export {name}") from exc
        function.restype = restype
        function.argtypes = list(argtypes)
    found = library.nkv_build_id().decode("utf-8", "replace")
    verify_build_id(found, path, override=override, source_dir=source_dir, include_dir=include_dir)
    return library


def load_library() -> ctypes.CDLL:
    """Return the loaded library, loading it on first use."""
    global _LIBRARY
    if _LIBRARY is not None:
        return _LIBRARY
    with _LOCK:
        if _LIBRARY is None:
            _LIBRARY = open_library(Path(library_path()),
                                    override=bool(os.environ.get("NANOKV_LIBRARY")))
    return _LIBRARY


_HOST_LOCK = Lock()
_HOST = None


def load_host():
    """The C++ host binding of the backend's per-call store and gather
    (``nanokv._nkv_host``), bound to the loaded library's entry points.  A
    missing or stale binding raises RuntimeError: there is no slower path
    to fall back to silently."""
    global _HOST
    if _HOST is not None:
        return _HOST
    library = load_library()
    with _HOST_LOCK:
        if _HOST is None:
            import importlib

            try:
                module = importlib.import_module("nanokv._nkv_host")
            except ImportError as exc:
                raise RuntimeError(
                    f"nanokv host binding not built or not loadable ({_build.host_module_path()}: "
                    f"{exc}); run __graft_entry__.build() or python -m nanokv.build") from exc
            source = _build.SOURCE_DIR / _build.HOST_SOURCE
            if source.is_file() and (_build.INCLUDE_DIR / "nanokv.h").is_file():
                expected = _build.host_build_id()
                if module.build_id() != expected:
                    raise RuntimeError(
                        f"{module.__file__} is stale: built as {module.build_id()!r}, the sources "
                        f"and this torch give {expected!r}; rebuild it (__graft_entry__.build() or "
                        "python -m nanokv.build)")

            def address(name: str) -> int:
                return ctypes.cast(getattr(library, name), ctypes.c_void_p).value

            module.bind(address("nkv_store"), address("nkv_gather"), address("nkv_last_error"))
            _HOST = module
    return _HOST


def build_id() -> str:
    """nkv_build_id() of the loaded library: the fingerprint of the sources
    it was built from and its launch-shape config."""
    return load_library().nkv_build_id().decode("utf-8", "replace")


def check(status: int, what: str) -> None:
    """Raise RuntimeError carrying nkv_last_error() when status != 0."""
    if status != 0:
        message = load_library().nkv_last_error()
        text = message.decode("utf-8", "replace") if message else ""
        raise RuntimeError(f"{what} failed (nkv status {status}): {text}")
