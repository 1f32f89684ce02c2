"""ctypes binding of ``libnanokv.so`` (the C ABI of ``include/nanokv.h``).

The library is loaded lazily, once, under a lock (the double-checked load of
the reference's CUDA backend, nanovllm/layers/paged_kv/cuda_backend.py:21-42).
A missing or unloadable library raises ``RuntimeError`` with the path and the
loader's message: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path
from threading import Lock

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
        (c_ptr, c_i64, c_i64, c_ptr, c_i64, c_ptr, c_ptr),
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


def load_library() -> ctypes.CDLL:
    """Return the loaded library, loading it on first use."""
    global _LIBRARY
    if _LIBRARY is not None:
        return _LIBRARY
    with _LOCK:
        if _LIBRARY is None:
            path = Path(library_path())
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
            _LIBRARY = library
    return _LIBRARY


def check(status: int, what: str) -> None:
    """Raise RuntimeError carrying nkv_last_error() when status != 0."""
    if status != 0:
        message = load_library().nkv_last_error()
        text = message.decode("utf-8", "replace") if message else ""
        raise RuntimeError(f"{what} failed (nkv status {status}): {text}")
