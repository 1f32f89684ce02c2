"""The ``hip`` paged-KV backend: the reference's backend protocol
(nanovllm/layers/paged_kv/base.py:38-65) implemented by the nanokv HIP
library for MI355X.

It mirrors the reference's CUDA backend (nanovllm/layers/paged_kv/
cuda_backend.py:31-104): validate with the shared validators, then run the
``nanovllm_paged_kv`` ops.  Loading registers the ops on the CUDA key (for
``torch.ops.nanovllm_paged_kv.*`` callers); the backend itself calls the
same implementations directly, without the dispatcher hop.  Loading is lazy
and lock-protected; a missing library raises instead of falling back to
another backend.
"""
from __future__ import annotations

from threading import Lock
from typing import Sequence

import torch

from nanokv import _lib
from nanokv.paged_kv import ops
from nanokv.paged_kv.base import (
    PagedKVAllocation,
    validate_store_inputs,
)

_LOAD_LOCK = Lock()
_READY = False
_HOST = None  # the C++ host binding, set by the first load


def hip_runtime_available() -> bool:
    """True on a ROCm build of PyTorch with a visible GPU."""
    return torch.version.hip is not None and torch.cuda.is_available()


def hip_extension_available() -> bool:
    """True when the built library and its host binding load, export the
    full ABI and match the sources (their build ids)."""
    try:
        _lib.load_host()
    except RuntimeError:
        return False
    return True


class AttentionPlan(tuple):
    """``(plan, first_part)`` of :meth:`HIPPagedKVBackend.build_attention_plan`,
    unpacked like the pair, with ``lengths`` = (total context rows, number
    of sequences, kv heads) it was built for: a plan splits those rows among
    the kernel's workers of each kv head, so it serves only contexts of the
    same lengths in caches with as many kv heads."""

    def __new__(cls, plan: torch.Tensor, first_part: torch.Tensor,
                lengths: tuple[int, int, int]):
        self = super().__new__(cls, (plan, first_part))
        self.lengths = lengths
        return self


def reset_hip_backend_state_for_tests() -> None:
    global _READY
    with _LOAD_LOCK:
        _READY = False


class HIPPagedKVBackend:
    name = "hip"

    @staticmethod
    def _load() -> None:
        global _READY, _HOST
        if _READY:
            return
        with _LOAD_LOCK:
            if not _READY:
                _lib.load_library()
                _HOST = _lib.load_host()
                ops.register_ops()
                _READY = True

    def allocate(
        self,
        shape: Sequence[int],
        *,
        dtype: torch.dtype,
        device: torch.device | str,
    ) -> PagedKVAllocation:
        """One device tensor for the whole [2, layers, blocks, block, heads,
        dim] cache (model_runner.py:657-674), owned by a native
        HIPPagedKVCache (cuda_backend.py:44-65); per-layer views of it are
        contiguous, which the kernels require."""
        resolved = torch.device(device)
        if resolved.type != "cuda":
            raise ValueError("HIP Paged KV allocation requires a ROCm (cuda) device")
        if dtype not in ops.DTYPE_CODES:
            raise ValueError(f"HIP Paged KV allocation does not support dtype {dtype}")
        if any(int(size) <= 0 for size in shape) or not shape:
            raise ValueError("HIP Paged KV allocation dimensions must be positive")
        self._load()
        from nanokv.paged_kv.owner import HIPPagedKVCache

        index = torch.cuda.current_device() if resolved.index is None else resolved.index
        owner = HIPPagedKVCache(list(shape), dtype, index)
        return PagedKVAllocation(owner.tensor(), owner)

    def copy_slots_async(self, allocation: PagedKVAllocation, host_slots: torch.Tensor) -> torch.Tensor:
        """cuda_backend.py:67-74: pinned host slot mapping -> device through
        the owner's transfer lane."""
        if allocation.owner is None:
            raise ValueError("HIP Paged KV allocation has no native owner")
        return allocation.owner.copy_slots_async(host_slots)

    # store and gather are called once per layer and, in the reference's SDPA
    # decode loop, twice per request per layer (attention.py:284-300).  On
    # MI355X a HIP launch alone costs ~3 us of host time, so the call runs in
    # the C++ host binding (csrc/nkv_host.cpp): the reference validator's
    # checks, in its order and with its messages, the output allocation and
    # the C-ABI launch, on the caller's current stream.

    def store(
        self,
        key: torch.Tensor,
        value: torch.Tensor,
        key_cache: torch.Tensor,
        value_cache: torch.Tensor,
        slot_mapping: torch.Tensor,
    ) -> None:
        if not _READY:
            self._load()
        index = key.get_device()
        _HOST.store(key, value, key_cache, value_cache, slot_mapping,
                    ops.stream_of(index) if index >= 0 else 0)

    def gather(
        self,
        cache: torch.Tensor,
        block_table: torch.Tensor,
        sequence_length: int,
    ) -> torch.Tensor:
        if not _READY:
            self._load()
        index = cache.get_device()
        return _HOST.gather(cache, block_table, sequence_length,
                            ops.stream_of(index) if index >= 0 else 0)

    def gather_varlen(
        self,
        key_cache: torch.Tensor,
        value_cache: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        total_tokens: int,
        *,
        plan: torch.Tensor | None = None,
        out: tuple[torch.Tensor, torch.Tensor] | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """K and V of every sequence in one launch: rows
        [cu_seqlens_k[i], cu_seqlens_k[i+1]) of the outputs equal
        ``gather(cache, block_tables[i], cu_seqlens_k[i+1]-cu_seqlens_k[i])``
        (the per-request loop of attention.py:250-259, 284-292).
        ``total_tokens`` must equal ``cu_seqlens_k[-1]``.  A ``plan`` from
        :meth:`build_gather_plan` (e.g. one per decode step, shared by all
        layers) skips the planning launch; ``out`` reuses output buffers."""
        validate_varlen_inputs(key_cache, value_cache, block_tables, cu_seqlens_k, total_tokens)
        self._load()
        if plan is None and out is None:
            return ops.gather_varlen(
                key_cache, value_cache, block_tables, cu_seqlens_k, total_tokens
            )
        if plan is None:
            plan = self.build_gather_plan(key_cache, block_tables, cu_seqlens_k, total_tokens)
        if out is None:
            key_out = torch.empty(
                (total_tokens, *key_cache.shape[2:]), dtype=key_cache.dtype, device=key_cache.device
            )
            out = (key_out, torch.empty_like(key_out))
        key_out, value_out = out
        if key_out.shape[0] < total_tokens or value_out.shape != key_out.shape:
            raise ValueError("varlen Gather outputs must hold total_tokens rows")
        ops.gather_varlen_planned(
            key_cache, value_cache, plan, key_out, value_out
        )
        return key_out, value_out

    def build_gather_plan(
        self,
        cache: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        total_tokens: int,
    ) -> torch.Tensor:
        """Chunk list for :meth:`gather_varlen`; valid for every cache with
        the shape and dtype of ``cache`` (all layers, K and V)."""
        self._load()
        num_blocks, block_size, heads, head_dim = cache.shape
        return ops.build_gather_plan(
            block_tables, cu_seqlens_k, total_tokens, num_blocks, block_size,
            heads * head_dim, cache.dtype,
        )

    def build_store_gather_plan(
        self,
        cache: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        num_tokens: int,
        total_tokens: int,
    ) -> torch.Tensor:
        """Plan of :meth:`store_gather` for one prefill step (valid for every
        layer's caches of the shape and dtype of ``cache``): each new
        token's context row and table-derived slot, and the chunks of every
        request's cached prefix.  ``num_tokens`` is the step's new-token
        count (rows of K/V and of slot_mapping, cu_seqlens_q[-1]) and
        ``total_tokens`` its context rows (cu_seqlens_k[-1]); the plan is
        laid out for them."""
        self._load()
        num_blocks, block_size, heads, head_dim = cache.shape
        return ops.build_store_gather_plan(
            block_tables, cu_seqlens_q, cu_seqlens_k, num_tokens, total_tokens,
            num_blocks, block_size, heads * head_dim, cache.dtype,
        )

    def store_gather(
        self,
        key: torch.Tensor,
        value: torch.Tensor,
        key_cache: torch.Tensor,
        value_cache: torch.Tensor,
        slot_mapping: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        total_tokens: int,
        *,
        plan: torch.Tensor | None = None,
        out: tuple[torch.Tensor, torch.Tensor] | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """The prefill step's store followed by the gather of every
        request's whole context (attention.py:87-93 then :250-259), in one
        launch: the caches end as :meth:`store` leaves them and the outputs
        equal :meth:`gather_varlen` over ``cu_seqlens_k`` afterwards.  Exact
        when no slot repeats, each token's slot is -1 or the slot of its own
        position in its request's block table (as prefill packing produces,
        model_runner.py:757-820), and no request's cached prefix holds a row
        this call stores.  The reference's scheduler guarantees the last: a
        block is hashed for prefix reuse only after the step that filled it
        (scheduler.py:196-200, block_manager.py:229-258).  ``plan`` from
        :meth:`build_store_gather_plan` (one per step, built for these token
        and context counts) skips the planning launch; ``out`` reuses output
        buffers."""
        validate_store_inputs(key, value, key_cache, value_cache, slot_mapping)
        validate_varlen_inputs(key_cache, value_cache, block_tables, cu_seqlens_k, total_tokens)
        if (cu_seqlens_q.dtype != torch.int32 or cu_seqlens_q.ndim != 1
                or cu_seqlens_q.numel() != cu_seqlens_k.numel()):
            raise ValueError("cu_seqlens_q must be int32 with one entry per request plus one")
        self._load()
        if plan is None:
            plan = self.build_store_gather_plan(key_cache, block_tables, cu_seqlens_q, cu_seqlens_k,
                                                key.shape[0], total_tokens)
        if out is None:
            key_out = torch.empty((total_tokens, *key_cache.shape[2:]), dtype=key_cache.dtype,
                                  device=key_cache.device)
            out = (key_out, torch.empty_like(key_out))
        if out[0].shape[0] != total_tokens or out[1].shape != out[0].shape:
            raise ValueError("store+gather outputs must hold total_tokens rows")
        ops.store_gather(key, value, key_cache, value_cache, slot_mapping, plan,
                         block_tables.shape[0], out[0], out[1])
        return out

    def build_attention_plan(
        self,
        cache: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        total_tokens: int,
    ) -> "AttentionPlan":
        """(plan, first_part) for :meth:`paged_attention_decode`: the
        contexts, in 16-row chunks laid end to end, split into equal ranges,
        one per worker wavefront of the kernel (1024 / Hkv per kv head of
        ``cache``).  It depends on the context lengths and the kv-head count
        only, so one plan serves every layer of a step (and every step with
        the same lengths)."""
        self._load()
        plan, first_part = ops.build_attention_plan(cu_seqlens_k, total_tokens, cache.shape[1],
                                                    cache.shape[2])
        return AttentionPlan(plan, first_part,
                             (int(total_tokens), int(cu_seqlens_k.numel()) - 1, int(cache.shape[2])))

    def paged_attention_decode(
        self,
        q: torch.Tensor,
        key_cache: torch.Tensor,
        value_cache: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        total_tokens: int,
        softmax_scale: float,
        *,
        plan: tuple[torch.Tensor, torch.Tensor] | None = None,
        out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Decode attention read straight from the paged caches: for each
        sequence i (context length cu_seqlens_k[i+1] - cu_seqlens_k[i]) and
        query head h, softmax(scale * q[i,h] K_i^T) V_i over kv head
        h // (Hq / Hkv).  The decode call of Attention.forward
        (flash_attn_with_kvcache, attention.py:122-130) with the numerics of
        SDPAAttention's decode branch (attention.py:284-300), without the
        gather.  q [B, Hq, 128] bf16 or fp16 (the caches' type) -> [B, Hq, 128]
        in that type."""
        validate_varlen_inputs(key_cache, value_cache, block_tables, cu_seqlens_k, total_tokens)
        if q.ndim != 3 or q.shape[0] != block_tables.shape[0]:
            raise ValueError("q must be [num_seqs, num_q_heads, head_dim] with one row per sequence")
        if q.device != key_cache.device:
            raise ValueError("q and the caches must be on the same device")
        self._load()
        if plan is None:
            plan = self.build_attention_plan(key_cache, cu_seqlens_k, total_tokens)
        else:
            built_for = getattr(plan, "lengths", None)
            here = (int(total_tokens), block_tables.shape[0], key_cache.shape[2])
            if built_for is not None and built_for != here:
                raise ValueError(f"attention plan was built for {built_for[0]} context rows over "
                                 f"{built_for[1]} sequences and {built_for[2]} kv heads, not "
                                 f"{here[0]} over {here[1]} and {here[2]}: build it with "
                                 "build_attention_plan for these lengths and this cache")
            need = int(_lib.load_library().nkv_attention_plan_capacity(
                total_tokens, block_tables.shape[0], key_cache.shape[1]))
            if plan[0].shape[0] < need:
                raise ValueError(f"attention plan has {plan[0].shape[0]} entries, "
                                 f"{block_tables.shape[0]} sequences need {need}: build it with "
                                 "build_attention_plan for these lengths")
        if out is None:
            out = torch.empty_like(q)
        ops.paged_attention_decode(
            q, key_cache, value_cache, block_tables, plan[0], plan[1], float(softmax_scale), out
        )
        return out

    def build_prefill_plan(self, q: torch.Tensor, key_cache: torch.Tensor,
                           cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor) -> torch.Tensor:
        """Query tiles for :meth:`paged_attention_prefill`, the tiles that see
        the most keys first; depends on the lengths and the head layout
        only, so one plan serves every layer of a step."""
        self._load()
        group = q.shape[1] // key_cache.shape[2]
        return ops.build_prefill_plan(cu_seqlens_q, cu_seqlens_k, q.shape[0], group)

    def paged_attention_prefill(
        self,
        q: torch.Tensor,
        key_cache: torch.Tensor,
        value_cache: torch.Tensor,
        block_tables: torch.Tensor,
        cu_seqlens_q: torch.Tensor,
        cu_seqlens_k: torch.Tensor,
        softmax_scale: float,
        *,
        total_context_tokens: int | None = None,
        plan: torch.Tensor | None = None,
        out: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Causal prefill attention read straight from the paged caches: the
        prefill call of Attention.forward (flash_attn_varlen_func with
        block_table, attention.py:95-116) with the numerics of SDPAAttention's
        prefill (attention.py:226-282).  Request i's queries are rows
        [cu_seqlens_q[i], cu_seqlens_q[i+1]) of q [Tq, Hq, 128] (bf16 or fp16, the
        caches' type); its
        context is the first Lk = cu_seqlens_k[i+1] - cu_seqlens_k[i] rows
        of its block table, the queries being the last Lq of them.
        ``total_context_tokens`` (= cu_seqlens_k[-1]) is only read by the
        host-side value checks of index validation (read from the device
        when not given)."""
        from nanokv.paged_kv.base import index_value_validation_enabled

        total = total_context_tokens
        if total is None:  # read it only when the (synchronising) value checks run anyway
            total = int(cu_seqlens_k[-1]) if index_value_validation_enabled(cu_seqlens_k) else 0
        validate_varlen_inputs(key_cache, value_cache, block_tables, cu_seqlens_k, int(total))
        if cu_seqlens_q.shape != cu_seqlens_k.shape:
            raise ValueError("cu_seqlens_q and cu_seqlens_k must have num_seqs + 1 entries each")
        if q.ndim != 3 or q.device != key_cache.device:
            raise ValueError("q must be [tokens, num_q_heads, head_dim] on the caches' device")
        self._load()
        if plan is None:
            plan = self.build_prefill_plan(q, key_cache, cu_seqlens_q, cu_seqlens_k)
        if out is None:
            out = torch.empty_like(q)
        ops.paged_attention_prefill(q, key_cache, value_cache, block_tables, cu_seqlens_q,
                                    cu_seqlens_k, plan, float(softmax_scale), out)
        return out


def validate_varlen_inputs(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    total_tokens: int,
) -> None:
    """Host-visible contract of gather_varlen, in the style of
    base.py:117-151: shapes, dtypes and devices always; index values only
    when index validation is enabled (it synchronises)."""
    if key_cache.ndim != 4 or key_cache.shape != value_cache.shape:
        raise ValueError("key and value cache shape must match [blocks, block, kv_heads, head_dim]")
    if key_cache.dtype != value_cache.dtype:
        raise ValueError("key and value caches must have matching dtype")
    if block_tables.dtype != torch.int32 or block_tables.ndim != 2:
        raise ValueError("block_tables must be a two-dimensional int32 tensor")
    if not block_tables.is_contiguous():
        raise ValueError("block_tables must be contiguous")
    if cu_seqlens_k.dtype != torch.int32 or cu_seqlens_k.ndim != 1 or not cu_seqlens_k.is_contiguous():
        raise ValueError("cu_seqlens_k must be a contiguous one-dimensional int32 tensor")
    if cu_seqlens_k.numel() != block_tables.shape[0] + 1:
        raise ValueError("cu_seqlens_k must have one entry more than block_tables has rows")
    devices = {t.device for t in (key_cache, value_cache, block_tables, cu_seqlens_k)}
    if len(devices) != 1:
        raise ValueError("all paged KV Gather tensors must be on the same device")
    if total_tokens < 0:
        raise ValueError("total_tokens must be non-negative")
    if not key_cache.is_cuda:
        raise ValueError("HIP Paged KV Gather requires ROCm device tensors")
    from nanokv.paged_kv.base import index_value_validation_enabled

    if cu_seqlens_k.numel() and index_value_validation_enabled(cu_seqlens_k):
        cu = cu_seqlens_k.cpu()
        lengths = cu[1:] - cu[:-1]
        if int(cu[0]) != 0 or bool((lengths < 0).any()) or int(cu[-1]) != total_tokens:
            raise ValueError("cu_seqlens_k must start at 0, be non-decreasing and end at total_tokens")
        block_size, num_blocks = key_cache.shape[1], key_cache.shape[0]
        needed = (lengths + block_size - 1) // block_size
        if bool((needed > block_tables.shape[1]).any()):
            raise ValueError("block_tables do not cover the requested sequence lengths")
        tables = block_tables.cpu()
        columns = torch.arange(tables.shape[1]).unsqueeze(0)
        used = columns < needed.unsqueeze(1)
        if bool((((tables < 0) | (tables >= num_blocks)) & used).any()):
            raise ValueError("block_tables contain an invalid physical block")
