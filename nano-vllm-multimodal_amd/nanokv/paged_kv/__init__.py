"""Paged-KV backend plugin API (the reference's nanovllm.layers.paged_kv,
nanovllm/layers/paged_kv/__init__.py:1-40) with the ``hip`` backend.

This package provides the ``hip`` backend only; ``pytorch``, ``triton`` and
``cuda`` stay with the host engine, whose ``create_paged_kv_backend`` gains a
``"hip"`` branch that returns :class:`HIPPagedKVBackend`.
"""
from __future__ import annotations

from nanokv.paged_kv.base import (
    BACKEND_NAMES,
    GatherDimensions,
    PagedKVAllocation,
    PagedKVBackend,
    StoreDimensions,
    index_value_validation_enabled,
    resolve_paged_kv_backend_name,
    validate_gather_inputs,
    validate_store_inputs,
)


def create_paged_kv_backend(name: str) -> PagedKVBackend:
    """__init__.py:15-28 for the ``hip`` name.  The other reference names
    are provided by the host engine and are rejected here with that reason;
    an unknown name raises as in the reference."""
    if name == "hip":
        from nanokv.paged_kv.hip_backend import HIPPagedKVBackend

        return HIPPagedKVBackend()
    if name in ("pytorch", "triton", "cuda"):
        raise ValueError(
            f"paged KV backend {name!r} belongs to the host engine "
            "(nanovllm.layers.paged_kv); nanokv provides 'hip'"
        )
    raise ValueError(f"unknown paged KV backend: {name}")


_DEFAULT_BACKEND = None


def store_kvcache(key, value, k_cache, v_cache, slot_mapping) -> None:
    """The legacy store entry point of the attention layer
    (nanovllm/layers/attention.py:10-33, hard-wired to the Triton backend
    there), on the ``hip`` backend: write this step's K/V rows [N, H, D]
    into the paged caches at slot_mapping, skipping -1.  Attention.forward
    calls it when no backend is bound and the caches are (:86-93)."""
    global _DEFAULT_BACKEND
    if _DEFAULT_BACKEND is None:
        _DEFAULT_BACKEND = create_paged_kv_backend("hip")
    _DEFAULT_BACKEND.store(key, value, k_cache, v_cache, slot_mapping)


__all__ = [
    "BACKEND_NAMES",
    "GatherDimensions",
    "PagedKVAllocation",
    "PagedKVBackend",
    "StoreDimensions",
    "create_paged_kv_backend",
    "index_value_validation_enabled",
    "resolve_paged_kv_backend_name",
    "store_kvcache",
    "validate_gather_inputs",
    "validate_store_inputs",
]
