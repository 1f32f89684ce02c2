"""Per-step attention metadata packed on the GPU.

The reference builds slot_mapping, cu_seqlens and the -1 padded
block_tables in Python loops over sequences and tokens, then ships each with
its own pinned host-to-device copy (ModelRunner.prepare_prefill /
prepare_decode / prepare_block_tables, nanovllm/engine/model_runner.py:
696-707, 727-938).  Here the scheduler's per-sequence state goes to the
device as ONE int32 buffer in CSR form and one kernel expands it
(nkv_pack_decode / nkv_pack_prefill).  The host keeps only O(num_seqs)
numpy work: validating the CSR arrays and the few scalars that size the
outputs (slot count, table width, max lengths), which it knows without
reading device memory.

The result is a :class:`Context` with the fields of the reference's
``nanovllm.utils.context.Context`` (context.py:5-16).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Iterable, Sequence

import numpy as np
import torch
from torch.autograd.graph import increment_version

from nanokv import _lib
from nanokv.paged_kv.ops import current_stream_handle


@dataclass(slots=True)
class Context:
    """Fields of nanovllm/utils/context.py:5-16, plus
    ``total_context_tokens`` = cu_seqlens_k[-1] known on the host, which
    sizes varlen gather outputs without a device read."""

    is_prefill: bool = False
    cu_seqlens_q: torch.Tensor | None = None
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: torch.Tensor | None = None
    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    full_context_lens: torch.Tensor | None = None
    query_start_lens: torch.Tensor | None = None
    total_context_tokens: int = 0


def _int32_array(values, name: str) -> np.ndarray:
    array = np.ascontiguousarray(np.asarray(values, dtype=np.int64))
    if array.ndim != 1:
        raise ValueError(f"{name} must be one-dimensional")
    if array.size and (array.min() < -(2**31) or array.max() >= 2**31):
        raise ValueError(f"{name} does not fit int32")
    return array.astype(np.int32)


@dataclass
class SequenceBatch:
    """Scheduler state of one step, per sequence, in CSR form (host int32):
    the Sequence fields the packers read (nanovllm/engine/sequence.py:
    98-119) with the block lists concatenated in ``block_ids`` and delimited
    by ``block_offsets`` [B+1]."""

    num_tokens: np.ndarray
    block_offsets: np.ndarray
    block_ids: np.ndarray
    num_prompt_tokens: np.ndarray | None = None
    num_cached_tokens: np.ndarray | None = None
    num_scheduled_tokens: np.ndarray | None = None

    def __post_init__(self) -> None:
        self.num_tokens = _int32_array(self.num_tokens, "num_tokens")
        self.block_offsets = _int32_array(self.block_offsets, "block_offsets")
        self.block_ids = _int32_array(self.block_ids, "block_ids")
        b = self.num_tokens.size
        for name in ("num_prompt_tokens", "num_cached_tokens", "num_scheduled_tokens"):
            value = getattr(self, name)
            if value is not None:
                value = _int32_array(value, name)
                if value.size != b:
                    raise ValueError(f"{name} must have one entry per sequence")
                setattr(self, name, value)
        if self.block_offsets.size != b + 1:
            raise ValueError("block_offsets must have num_seqs + 1 entries")
        if self.block_offsets[0] != 0 or self.block_offsets[-1] != self.block_ids.size:
            raise ValueError("block_offsets must start at 0 and end at len(block_ids)")
        if b and bool((np.diff(self.block_offsets) < 0).any()):
            raise ValueError("block_offsets must be non-decreasing")

    @property
    def num_seqs(self) -> int:
        return int(self.num_tokens.size)

    @property
    def block_counts(self) -> np.ndarray:
        return np.diff(self.block_offsets)

    @classmethod
    def from_block_lists(
        cls,
        num_tokens: Iterable[int],
        block_tables: Sequence[Sequence[int]],
        *,
        num_prompt_tokens=None,
        num_cached_tokens=None,
        num_scheduled_tokens=None,
    ) -> "SequenceBatch":
        lengths = [len(table) for table in block_tables]
        offsets = np.zeros(len(lengths) + 1, dtype=np.int64)
        np.cumsum(lengths, out=offsets[1:])
        ids = (
            np.concatenate([np.asarray(t, dtype=np.int64) for t in block_tables if len(t)])
            if any(lengths)
            else np.zeros(0, dtype=np.int64)
        )
        return cls(
            np.asarray(list(num_tokens)), offsets, ids, num_prompt_tokens,
            num_cached_tokens, num_scheduled_tokens,
        )

    @classmethod
    def from_sequences(cls, seqs: Sequence[object]) -> "SequenceBatch":
        """From objects with the reference Sequence attributes
        (len(), block_table, num_prompt_tokens, num_cached_tokens,
        num_scheduled_tokens)."""
        return cls.from_block_lists(
            [len(s) for s in seqs],
            [s.block_table for s in seqs],
            num_prompt_tokens=[getattr(s, "num_prompt_tokens", 0) for s in seqs],
            num_cached_tokens=[getattr(s, "num_cached_tokens", 0) for s in seqs],
            num_scheduled_tokens=[getattr(s, "num_scheduled_tokens", 0) for s in seqs],
        )


@dataclass
class DecodeGraphBuffers:
    """Fixed-address decode metadata for a captured decode graph: the
    buffers of ModelRunner.capture_cudagraph (model_runner.py:1093-1106,
    zero-initialised like them) plus cu_seqlens_k for a varlen gather.
    A graph captured for batch bucket ``bs`` reads the first ``bs`` rows."""

    slot_mapping: torch.Tensor   # [max_num_seqs] int32
    context_lens: torch.Tensor   # [max_num_seqs] int32
    block_tables: torch.Tensor   # [max_num_seqs, max_blocks] int32
    cu_seqlens_k: torch.Tensor   # [max_num_seqs + 1] int32

    @classmethod
    def allocate(cls, device: torch.device | str, max_num_seqs: int, max_blocks: int) -> "DecodeGraphBuffers":
        if max_num_seqs <= 0 or max_blocks <= 0:
            raise ValueError("max_num_seqs and max_blocks must be positive")
        if max_num_seqs > _lib.NKV_MAX_PACK_SEQS:
            raise ValueError(f"at most {_lib.NKV_MAX_PACK_SEQS} sequences per decode graph")
        device = torch.device(device)
        zeros = lambda *shape: torch.zeros(shape, dtype=torch.int32, device=device)  # noqa: E731
        return cls(zeros(max_num_seqs), zeros(max_num_seqs), zeros(max_num_seqs, max_blocks),
                   zeros(max_num_seqs + 1))

    @property
    def max_num_seqs(self) -> int:
        return int(self.slot_mapping.numel())

    @property
    def max_blocks(self) -> int:
        return int(self.block_tables.shape[1])

    @property
    def device(self) -> torch.device:
        return self.slot_mapping.device


class DevicePacker:
    """Launches the packing kernels for one device and block size.

    Host inputs are staged in one pinned int32 buffer that is reused across
    calls; an event recorded after each upload guards the reuse (the
    buffer is rewritten only once the previous copy has finished), the
    role the reference's PagedKVCache transfer events play
    (csrc/paged_kv/paged_kv.cpp:137-147).
    """

    def __init__(self, device: torch.device | str, block_size: int) -> None:
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("DevicePacker requires a ROCm (cuda) device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.block_size = int(block_size)
        self._staging: torch.Tensor | None = None
        self._uploaded: torch.cuda.Event | None = None
        _lib.load_library()

    # ------------------------------------------------------------ staging
    def _upload(self, parts: Sequence[np.ndarray]) -> list[torch.Tensor]:
        sizes = [int(p.size) for p in parts]
        total = max(1, sum(sizes))
        if self._uploaded is not None:
            self._uploaded.synchronize()
        if self._staging is None or self._staging.numel() < total:
            self._staging = torch.empty(max(total, 1024), dtype=torch.int32, pin_memory=True)
        host = self._staging.numpy()
        offset = 0
        for part, size in zip(parts, sizes):
            host[offset : offset + size] = part
            offset += size
        device_buffer = torch.empty(total, dtype=torch.int32, device=self.device)
        device_buffer.copy_(self._staging[:total], non_blocking=True)
        if self._uploaded is None:
            self._uploaded = torch.cuda.Event()
        self._uploaded.record(torch.cuda.current_stream(self.device))
        views, offset = [], 0
        for size in sizes:
            views.append(device_buffer[offset : offset + size])
            offset += size
        return views

    def _stream(self) -> int:
        return current_stream_handle(self.device)

    @staticmethod
    def _width(batch: SequenceBatch, table_width: int | None) -> int:
        longest = int(batch.block_counts.max()) if batch.num_seqs else 0
        if table_width is None:
            return longest
        if table_width < longest:
            raise ValueError("table_width is smaller than the longest block list")
        return int(table_width)

    @staticmethod
    def _check_num_seqs(batch: SequenceBatch) -> None:
        if batch.num_seqs > _lib.NKV_MAX_PACK_SEQS:
            raise ValueError(
                f"device packing supports at most {_lib.NKV_MAX_PACK_SEQS} sequences per step"
            )

    # ------------------------------------------------------------- decode
    def pack_decode(self, batch: SequenceBatch, *, table_width: int | None = None) -> Context:
        """model_runner.py:892-938: slot of the last token of every sequence,
        context_lens, -1 padded block_tables, plus cu_seqlens_k."""
        self._check_num_seqs(batch)
        b = batch.num_seqs
        if b and bool((batch.block_counts < 1).any()):
            raise ValueError("every decoding sequence needs a non-empty block_table")
        if b and bool((batch.num_tokens < 1).any()):
            raise ValueError("every decoding sequence needs at least one token")
        width = self._width(batch, table_width)
        d_tokens, d_offsets, d_ids = self._upload(
            [batch.num_tokens, batch.block_offsets, batch.block_ids]
        )
        out = torch.empty(3 * b + 1 + b * width, dtype=torch.int32, device=self.device)
        slots = out[:b]
        context_lens = out[b : 2 * b]
        cu_seqlens_k = out[2 * b : 3 * b + 1]
        tables = out[3 * b + 1 :].view(b, width)
        status = _lib.load_library().nkv_pack_decode(
            d_tokens.data_ptr(), d_offsets.data_ptr(), d_ids.data_ptr() if d_ids.numel() else None,
            d_ids.numel(), b, b, self.block_size, width, width, slots.data_ptr(),
            context_lens.data_ptr(), tables.data_ptr() if tables.numel() else None,
            cu_seqlens_k.data_ptr(), self._stream(),
        )
        _lib.check(status, "nkv_pack_decode")
        total = int(batch.num_tokens.astype(np.int64).sum())
        return Context(
            is_prefill=False,
            cu_seqlens_k=cu_seqlens_k,
            max_seqlen_k=int(batch.num_tokens.max()) if b else 0,
            slot_mapping=slots,
            context_lens=context_lens,
            block_tables=tables,
            total_context_tokens=total,
        )

    def pack_decode_into(
        self,
        batch: SequenceBatch,
        buffers: "DecodeGraphBuffers",
        *,
        padded_seqs: int | None = None,
    ) -> Context:
        """Decode packing straight into the fixed-address buffers a captured
        decode graph reads.  Equals the reference's replay fill
        (model_runner.py:993-1011): slot_mapping[bs:padded] = -1,
        context_lens[bs:padded] = 0, block_tables[:bs, :w] = the -1 padded
        tables with w = the longest block list of the batch, while columns
        >= w and rows >= bs keep their contents.  ``padded`` defaults to the
        buffers' capacity (the reference fills the whole max_bs buffers).
        One kernel, no fills or device-to-device copies, capturable."""
        self._check_num_seqs(batch)
        b = batch.num_seqs
        padded = buffers.max_num_seqs if padded_seqs is None else int(padded_seqs)
        if not b <= padded <= buffers.max_num_seqs:
            raise ValueError("padded_seqs must be in [num_seqs, buffers.max_num_seqs]")
        if b and bool((batch.block_counts < 1).any()):
            raise ValueError("every decoding sequence needs a non-empty block_table")
        if b and bool((batch.num_tokens < 1).any()):
            raise ValueError("every decoding sequence needs at least one token")
        width = self._width(batch, None)
        if width > buffers.max_blocks:
            raise ValueError("a block list is longer than the graph buffers' max_blocks")
        if buffers.device != self.device:
            raise ValueError("graph buffers live on another device")
        d_tokens, d_offsets, d_ids = self._upload(
            [batch.num_tokens, batch.block_offsets, batch.block_ids]
        )
        status = _lib.load_library().nkv_pack_decode(
            d_tokens.data_ptr(), d_offsets.data_ptr(), d_ids.data_ptr() if d_ids.numel() else None,
            d_ids.numel(), b, padded, self.block_size, width, buffers.max_blocks,
            buffers.slot_mapping.data_ptr(), buffers.context_lens.data_ptr(),
            buffers.block_tables.data_ptr(), buffers.cu_seqlens_k.data_ptr(), self._stream(),
        )
        _lib.check(status, "nkv_pack_decode")
        # The kernel wrote the buffers behind torch's back: bump their version
        # counters, so whatever keys a cache on a tensor's version (the decode
        # plan of nanokv.flash) sees the new contents.
        for written in (buffers.slot_mapping, buffers.context_lens, buffers.block_tables,
                        buffers.cu_seqlens_k):
            increment_version(written)
        return Context(
            is_prefill=False,
            cu_seqlens_k=buffers.cu_seqlens_k[: b + 1],
            max_seqlen_k=int(batch.num_tokens.max()) if b else 0,
            slot_mapping=buffers.slot_mapping[:b],
            context_lens=buffers.context_lens[:b],
            block_tables=buffers.block_tables[:b],
            total_context_tokens=int(batch.num_tokens.astype(np.int64).sum()),
        )

    def pack_decode_pool(self, pool, seq_slots, num_tokens, *,
                         table_width: int | None = None) -> Context:
        """pack_decode with each sequence's block list read from the device
        block pool (table of slot seq_slots[i]) instead of an uploaded CSR:
        only the slots and token counts travel.  The tables are padded to
        the longest list, ceil(num_tokens / block_size) blocks, as
        prepare_block_tables pads (model_runner.py:696-707)."""
        slots_h = _int32_array(seq_slots, "seq_slots")
        tokens_h = _int32_array(num_tokens, "num_tokens")
        b = int(slots_h.size)
        if tokens_h.size != b:
            raise ValueError("seq_slots and num_tokens must have one entry per sequence")
        if b > _lib.NKV_MAX_PACK_SEQS:
            raise ValueError(f"device packing supports at most {_lib.NKV_MAX_PACK_SEQS} sequences per step")
        if b and bool((tokens_h < 1).any()):
            raise ValueError("every decoding sequence needs at least one token")
        if b and (bool((slots_h < 0).any()) or bool((slots_h >= pool.max_seqs).any())):
            raise ValueError("seq_slots must name slots of the pool")
        if pool.block_size != self.block_size or pool.device != self.device:
            raise ValueError("the pool has another block size or device")
        longest = int(((tokens_h.astype(np.int64) + self.block_size - 1) // self.block_size).max()) if b else 0
        width = longest if table_width is None else int(table_width)
        if width < longest or width > pool.width:
            raise ValueError("table_width must cover the longest block list and fit the pool")
        d_tokens, d_slots = self._upload([tokens_h, slots_h])
        out = torch.empty(3 * b + 1 + b * width, dtype=torch.int32, device=self.device)
        slots = out[:b]
        context_lens = out[b: 2 * b]
        cu_seqlens_k = out[2 * b: 3 * b + 1]
        tables = out[3 * b + 1:].view(b, width)
        status = _lib.load_library().nkv_pack_decode_pool(
            ctypes.byref(pool.desc), d_tokens.data_ptr(), d_slots.data_ptr(), b, b, self.block_size,
            width, width, slots.data_ptr(), context_lens.data_ptr(),
            tables.data_ptr() if tables.numel() else None, cu_seqlens_k.data_ptr(), self._stream(),
        )
        _lib.check(status, "nkv_pack_decode_pool")
        return Context(
            is_prefill=False,
            cu_seqlens_k=cu_seqlens_k,
            max_seqlen_k=int(tokens_h.max()) if b else 0,
            slot_mapping=slots,
            context_lens=context_lens,
            block_tables=tables,
            total_context_tokens=int(tokens_h.astype(np.int64).sum()),
        )

    def pack_prefill_pool(self, pool, seq_slots, num_cached_tokens, num_scheduled_tokens,
                          num_prompt_tokens=None, *, table_width: int | None = None,
                          force_block_tables: bool = False) -> Context:
        """pack_prefill with each sequence's block list read from the device
        block pool.  A sequence's list covers its whole prompt (allocate
        takes ceil(len / block_size) blocks), so the host checks coverage
        from the token counts; the tables are padded to the longest list."""
        slots_h = _int32_array(seq_slots, "seq_slots")
        cached_h = _int32_array(num_cached_tokens, "num_cached_tokens")
        sched_h = _int32_array(num_scheduled_tokens, "num_scheduled_tokens")
        b = int(slots_h.size)
        if cached_h.size != b or sched_h.size != b:
            raise ValueError("one entry per sequence in every array")
        if b > _lib.NKV_MAX_PACK_SEQS:
            raise ValueError(f"device packing supports at most {_lib.NKV_MAX_PACK_SEQS} sequences per step")
        if b and (bool((cached_h < 0).any()) or bool((sched_h < 0).any())):
            raise ValueError("cached and scheduled token counts must be non-negative")
        if b and (bool((slots_h < 0).any()) or bool((slots_h >= pool.max_seqs).any())):
            raise ValueError("seq_slots must name slots of the pool")
        if pool.block_size != self.block_size or pool.device != self.device:
            raise ValueError("the pool has another block size or device")
        ends = cached_h.astype(np.int64) + sched_h
        prompt_h = (_int32_array(num_prompt_tokens, "num_prompt_tokens")
                    if num_prompt_tokens is not None else ends.astype(np.int32))
        if prompt_h.size != b:
            raise ValueError("one entry per sequence in every array")
        blocks = (np.maximum(prompt_h.astype(np.int64), ends) + self.block_size - 1) // self.block_size
        num_slots = int(sched_h.astype(np.int64).sum())
        with_tables = force_block_tables or int(cached_h.astype(np.int64).sum()) > 0
        longest = int(blocks.max()) if b else 0
        width = (longest if table_width is None else int(table_width)) if with_tables else 0
        if with_tables and (width < longest or width > pool.width):
            raise ValueError("table_width must cover the longest block list and fit the pool")
        d_cached, d_sched, d_prompt, d_slots = self._upload([cached_h, sched_h, prompt_h, slots_h])
        sizes = [b + 1, b + 1, num_slots, b * width, b, b, 2]
        out = torch.empty(sum(sizes), dtype=torch.int32, device=self.device)
        views, offset = [], 0
        for size in sizes:
            views.append(out[offset: offset + size])
            offset += size
        cu_q, cu_k, slots, tables, full_ctx, q_start, max_lens = views
        tables = tables.view(b, width) if with_tables else None
        status = _lib.load_library().nkv_pack_prefill_pool(
            ctypes.byref(pool.desc), d_cached.data_ptr(), d_sched.data_ptr(), d_prompt.data_ptr(),
            d_slots.data_ptr(), b, self.block_size, width, num_slots, cu_q.data_ptr(),
            cu_k.data_ptr(), slots.data_ptr() if num_slots else None,
            tables.data_ptr() if tables is not None and tables.numel() else None,
            full_ctx.data_ptr(), q_start.data_ptr(), max_lens.data_ptr(), self._stream(),
        )
        _lib.check(status, "nkv_pack_prefill_pool")
        return Context(
            is_prefill=True,
            cu_seqlens_q=cu_q,
            cu_seqlens_k=cu_k,
            max_seqlen_q=int(sched_h.max()) if b else 0,
            max_seqlen_k=int(ends.max()) if b else 0,
            slot_mapping=slots,
            block_tables=tables,
            full_context_lens=full_ctx,
            query_start_lens=q_start,
            total_context_tokens=int(ends.sum()),
        )

    # ------------------------------------------------------------ prefill
    def pack_prefill(
        self,
        batch: SequenceBatch,
        *,
        table_width: int | None = None,
        force_block_tables: bool = False,
    ) -> Context:
        """model_runner.py:757-820, 856-882: cu_seqlens_q/k, slot_mapping of
        the scheduled positions, full_context_lens, query_start_lens and,
        when some sequence has cached tokens (cu_seqlens_k[-1] >
        cu_seqlens_q[-1]) or ``force_block_tables``, the block_tables."""
        self._check_num_seqs(batch)
        if batch.num_cached_tokens is None or batch.num_scheduled_tokens is None:
            raise ValueError("prefill packing needs num_cached_tokens and num_scheduled_tokens")
        b = batch.num_seqs
        cached = batch.num_cached_tokens.astype(np.int64)
        scheduled = batch.num_scheduled_tokens.astype(np.int64)
        if b and (bool((cached < 0).any()) or bool((scheduled < 0).any())):
            raise ValueError("cached and scheduled token counts must be non-negative")
        counts = batch.block_counts.astype(np.int64)
        ends = cached + scheduled
        has_blocks = counts > 0
        needed = (ends + self.block_size - 1) // self.block_size
        if bool((has_blocks & (needed > counts)).any()):
            raise ValueError("a block_table does not cover its scheduled tokens")
        num_slots = int(scheduled[has_blocks].sum())
        with_tables = force_block_tables or int(cached.sum()) > 0
        width = self._width(batch, table_width) if with_tables else 0
        prompt = batch.num_prompt_tokens if batch.num_prompt_tokens is not None else ends.astype(np.int32)
        d_cached, d_sched, d_prompt, d_offsets, d_ids = self._upload(
            [batch.num_cached_tokens, batch.num_scheduled_tokens, prompt, batch.block_offsets,
             batch.block_ids]
        )
        sizes = [b + 1, b + 1, num_slots, b * width, b, b, 2]
        out = torch.empty(sum(sizes), dtype=torch.int32, device=self.device)
        views, offset = [], 0
        for size in sizes:
            views.append(out[offset : offset + size])
            offset += size
        cu_q, cu_k, slots, tables, full_ctx, q_start, max_lens = views
        tables = tables.view(b, width) if with_tables else None
        status = _lib.load_library().nkv_pack_prefill(
            d_cached.data_ptr(), d_sched.data_ptr(), d_prompt.data_ptr(), d_offsets.data_ptr(),
            d_ids.data_ptr() if d_ids.numel() else None, d_ids.numel(), b, self.block_size,
            width, num_slots, cu_q.data_ptr(), cu_k.data_ptr(),
            slots.data_ptr() if num_slots else None,
            tables.data_ptr() if tables is not None and tables.numel() else None,
            full_ctx.data_ptr(), q_start.data_ptr(), max_lens.data_ptr(), self._stream(),
        )
        _lib.check(status, "nkv_pack_prefill")
        return Context(
            is_prefill=True,
            cu_seqlens_q=cu_q,
            cu_seqlens_k=cu_k,
            max_seqlen_q=int(scheduled.max()) if b else 0,
            max_seqlen_k=int(ends.max()) if b else 0,
            slot_mapping=slots,
            block_tables=tables,
            full_context_lens=full_ctx,
            query_start_lens=q_start,
            total_context_tokens=int(ends.sum()),
        )
