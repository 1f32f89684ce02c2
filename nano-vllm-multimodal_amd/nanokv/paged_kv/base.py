"""Paged-KV backend contract: dimension records, the backend protocol, the
host-side input validators and backend-name resolution.

Restates nanovllm/layers/paged_kv/base.py:10-170 of the reference.  The
checks, their order and the ValueError message substrings are the
reference's, because callers and the reference's own tests match on them
(tests/test_paged_kv_backends.py:40-124); ``resolve_paged_kv_backend_name``
adds the ``hip`` backend.
"""
from __future__ import annotations

import os
from dataclasses import dataclass
from typing import Protocol, Sequence

import torch

VALIDATE_INDICES_ENV = "NANOVLLM_PAGED_KV_VALIDATE_INDICES"
BACKEND_NAMES = ("auto", "pytorch", "triton", "cuda", "hip")


@dataclass(frozen=True, slots=True)
class StoreDimensions:
    """base.py:10-20."""

    num_tokens: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int

    @property
    def num_slots(self) -> int:
        return self.num_blocks * self.block_size


@dataclass(frozen=True, slots=True)
class GatherDimensions:
    """base.py:23-29."""

    sequence_length: int
    required_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int


@dataclass(slots=True)
class PagedKVAllocation:
    """base.py:32-35: the cache tensor and an optional native owner that the
    model runner keeps alive."""

    tensor: torch.Tensor
    owner: object | None = None


class PagedKVBackend(Protocol):
    """base.py:38-65."""

    name: str

    def allocate(
        self, shape: Sequence[int], *, dtype: torch.dtype, device: torch.device | str
    ) -> PagedKVAllocation: ...

    def store(
        self,
        key: torch.Tensor,
        value: torch.Tensor,
        key_cache: torch.Tensor,
        value_cache: torch.Tensor,
        slot_mapping: torch.Tensor,
    ) -> None: ...

    def gather(
        self, cache: torch.Tensor, block_table: torch.Tensor, sequence_length: int
    ) -> torch.Tensor: ...


def index_value_validation_enabled(tensor: torch.Tensor) -> bool:
    """base.py:68-72: index values in host memory are always range-checked;
    device-resident ones only when the opt-in debug variable is set, because
    the check synchronises with the device."""
    if not tensor.is_cuda:
        return True
    flag = os.environ.get(VALIDATE_INDICES_ENV, "0").strip().lower()
    return flag in ("1", "true", "yes", "on")


def _same_device(a: torch.Tensor, b: torch.Tensor) -> bool:
    """``a.device == b.device`` without building device objects: GPU tensors
    compare by index; host-side ones (index -1) fall back to the devices."""
    index = a.get_device()
    if index != b.get_device():
        return False
    return index >= 0 or a.device == b.device


def check_store_inputs(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """The checks of base.py:75-114, in its order and with its messages,
    without building the StoreDimensions record (the per-call path of the
    hip backend; :func:`validate_store_inputs` wraps it)."""
    kshape = key.shape
    if key.ndim != 3 or value.ndim != 3 or kshape != value.shape:
        raise ValueError("key and value must have matching shape [tokens, kv_heads, head_dim]")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("key and value inner dimensions must be contiguous")
    cshape = key_cache.shape
    if key_cache.ndim != 4 or value_cache.ndim != 4 or cshape != value_cache.shape:
        raise ValueError("key and value cache shape must match [blocks, block, kv_heads, head_dim]")
    if cshape[2] != kshape[1] or cshape[3] != kshape[2]:
        raise ValueError("cache shape does not match key/value kv_heads and head_dim")
    if not (_same_device(key, value) and _same_device(key, key_cache)
            and _same_device(key, value_cache) and _same_device(key, slot_mapping)):
        raise ValueError("all paged KV Store tensors must be on the same device")
    dtype = key.dtype
    if not (dtype == value.dtype == key_cache.dtype == value_cache.dtype):
        raise ValueError("key, value, and caches must have matching dtype")
    if slot_mapping.dtype != torch.int32 or slot_mapping.ndim != 1:
        raise ValueError("slot_mapping must be a one-dimensional int32 tensor")
    num_tokens = kshape[0]
    if slot_mapping.shape[0] != num_tokens:
        raise ValueError("slot_mapping length must equal the number of input tokens")
    if not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be contiguous")
    if num_tokens and index_value_validation_enabled(slot_mapping):
        num_slots = cshape[0] * cshape[1]
        out_of_range = (slot_mapping < -1) | (slot_mapping >= num_slots)
        if bool(out_of_range.any()):
            raise ValueError(f"slot_mapping contains a slot outside [-1, {num_slots})")


def validate_store_inputs(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> StoreDimensions:
    """base.py:75-114."""
    check_store_inputs(key, value, key_cache, value_cache, slot_mapping)
    num_tokens, num_kv_heads, head_dim = key.shape
    num_blocks, block_size = key_cache.shape[:2]
    return StoreDimensions(num_tokens, num_blocks, block_size, num_kv_heads, head_dim)


def check_gather_inputs(cache: torch.Tensor, block_table: torch.Tensor, sequence_length: int) -> int:
    """The checks of base.py:117-151, in its order and with its messages;
    returns the required block count without building the GatherDimensions
    record (the per-call path of the hip backend; :func:`validate_gather_inputs`
    wraps it).  The table prefix is sliced only when index values are
    checked."""
    if cache.ndim != 4:
        raise ValueError("cache must have shape [blocks, block, kv_heads, head_dim]")
    if cache.stride(-1) != 1:
        raise ValueError("cache inner dimensions must be contiguous")
    if block_table.dtype != torch.int32 or block_table.ndim != 1:
        raise ValueError("block_table must be a one-dimensional int32 tensor")
    if not _same_device(block_table, cache):
        raise ValueError("cache and block_table must be on the same device")
    if not block_table.is_contiguous():
        raise ValueError("block_table must be contiguous")
    if sequence_length < 0:
        raise ValueError("sequence_length must be non-negative")
    block_size = cache.shape[1]
    required_blocks = -(-sequence_length // block_size)
    if block_table.shape[0] < required_blocks:
        raise ValueError("block_table does not cover the requested sequence length")
    if required_blocks and index_value_validation_enabled(block_table):
        used = block_table[:required_blocks]
        if bool(((used < 0) | (used >= cache.shape[0])).any()):
            raise ValueError("block_table contains an invalid physical block")
    return required_blocks


def validate_gather_inputs(
    cache: torch.Tensor, block_table: torch.Tensor, sequence_length: int
) -> GatherDimensions:
    """base.py:117-151."""
    required_blocks = check_gather_inputs(cache, block_table, sequence_length)
    _, block_size, num_kv_heads, head_dim = cache.shape
    return GatherDimensions(sequence_length, required_blocks, block_size, num_kv_heads, head_dim)


def resolve_paged_kv_backend_name(
    requested: str,
    *,
    cuda_available: bool,
    cuda_extension_available: bool,
    hip_available: bool = False,
    hip_extension_available: bool = False,
) -> str:
    """base.py:154-170 plus ``hip``.  ``auto`` picks ``hip`` on a ROCm build
    with a visible GPU and a loadable nanokv library, then the reference's
    order (cuda extension, triton, pytorch).  An explicit name is returned
    unchanged: selection never falls back silently."""
    if requested not in BACKEND_NAMES:
        raise ValueError("paged_kv_backend must be one of: " + ", ".join(BACKEND_NAMES))
    if requested != "auto":
        return requested
    if hip_available and hip_extension_available:
        return "hip"
    if cuda_available and cuda_extension_available:
        return "cuda"
    if cuda_available:
        return "triton"
    return "pytorch"
