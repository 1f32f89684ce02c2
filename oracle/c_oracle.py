"""ctypes wrapper of the oracle's C restatement (oracle/nkv_oracle.c).

TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's
cpu_baseline leg).  Functions take numpy arrays; K/V/cache arrays may have
any element type (bf16 data is passed as int16 views).
"""
from __future__ import annotations

import ctypes
import os
from threading import Lock

import numpy as np

from oracle.build import LIBRARY_PATH, build

_LOCK = Lock()
_LIB = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int


def library():
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                if not LIBRARY_PATH.is_file():
                    build()
                lib = ctypes.CDLL(str(LIBRARY_PATH))
                lib.nkvo_store.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I]
                lib.nkvo_gather.argtypes = [_P, _P, _I64, _I64, _I64, _P, _I]
                lib.nkvo_gather_varlen.argtypes = [_P, _P, _I64, _P, _I64, _I64, _I64, _P, _I]
                lib.nkvo_pack_decode.argtypes = [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P]
                lib.nkvo_pack_prefill.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _P]
                lib.nkvo_max_threads.restype = _I
                for fn in ("nkvo_store", "nkvo_gather", "nkvo_gather_varlen",
                           "nkvo_pack_decode", "nkvo_pack_prefill"):
                    getattr(lib, fn).restype = None
                _LIB = lib
    return _LIB


def default_threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def _ptr(array: np.ndarray) -> int:
    return array.ctypes.data


def _i32(array) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(array, dtype=np.int32))


def store(key, value, key_cache, value_cache, slot_mapping, threads: int = 1) -> None:
    """In-place store; key/value [T, ...] may be row-strided views."""
    assert key_cache.flags.c_contiguous and value_cache.flags.c_contiguous
    row_bytes = key_cache.strides[1]
    slots = _i32(slot_mapping)
    library().nkvo_store(
        _ptr(key), _ptr(value), _ptr(key_cache), _ptr(value_cache), _ptr(slots),
        key.shape[0], key.strides[0], value.strides[0], row_bytes, threads,
    )


def gather(cache, block_table, sequence_length: int, threads: int = 1) -> np.ndarray:
    assert cache.flags.c_contiguous
    table = _i32(block_table)
    out = np.empty((sequence_length, *cache.shape[2:]), dtype=cache.dtype)
    if sequence_length:
        library().nkvo_gather(
            _ptr(cache), _ptr(table), sequence_length, cache.shape[1], cache.strides[1],
            _ptr(out), threads,
        )
    return out


def gather_varlen(cache, block_tables, cu_seqlens_k, threads: int = 1, out=None) -> np.ndarray:
    assert cache.flags.c_contiguous
    tables = _i32(block_tables)
    cu = _i32(cu_seqlens_k)
    total = int(cu[-1])
    if out is None:
        out = np.empty((total, *cache.shape[2:]), dtype=cache.dtype)
    if total:
        library().nkvo_gather_varlen(
            _ptr(cache), _ptr(tables), tables.shape[1], _ptr(cu), len(cu) - 1,
            cache.shape[1], cache.strides[1], _ptr(out), threads,
        )
    return out


def pack_decode(num_tokens, offsets, ids, block_size: int, width: int) -> dict:
    num_tokens, offsets, ids = _i32(num_tokens), _i32(offsets), _i32(ids)
    b = len(num_tokens)
    out = {
        "slot_mapping": np.empty(b, np.int32),
        "context_lens": np.empty(b, np.int32),
        "block_tables": np.empty((b, width), np.int32),
        "cu_seqlens_k": np.empty(b + 1, np.int32),
    }
    library().nkvo_pack_decode(
        _ptr(num_tokens), _ptr(offsets), _ptr(ids) if ids.size else None, b, block_size, width,
        _ptr(out["slot_mapping"]), _ptr(out["context_lens"]), _ptr(out["block_tables"]),
        _ptr(out["cu_seqlens_k"]),
    )
    return out


def pack_prefill(num_cached, num_scheduled, offsets, ids, block_size: int, width: int,
                 with_tables: bool = True) -> dict:
    num_cached, num_scheduled = _i32(num_cached), _i32(num_scheduled)
    offsets, ids = _i32(offsets), _i32(ids)
    b = len(num_cached)
    counts = offsets[1:] - offsets[:-1]
    total_slots = int(num_scheduled[counts > 0].sum())
    out = {
        "cu_seqlens_q": np.empty(b + 1, np.int32),
        "cu_seqlens_k": np.empty(b + 1, np.int32),
        "slot_mapping": np.empty(total_slots, np.int32),
        "block_tables": np.empty((b, width), np.int32) if with_tables else None,
    }
    library().nkvo_pack_prefill(
        _ptr(num_cached), _ptr(num_scheduled), _ptr(offsets), _ptr(ids) if ids.size else None,
        b, block_size, width, _ptr(out["cu_seqlens_q"]), _ptr(out["cu_seqlens_k"]),
        _ptr(out["slot_mapping"]) if total_slots else None,
        _ptr(out["block_tables"]) if with_tables else None,
    )
    return out
