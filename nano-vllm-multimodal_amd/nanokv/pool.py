"""Device block pool: the block bookkeeping of the reference BlockManager
(free-block FIFO, reference counts, per-sequence block tables;
nanovllm/engine/block_manager.py:87-118, 185-236) resident in HBM.

The scheduler keeps making its decisions as the reference does; every
BlockManager call it makes is recorded here, in the same order, and
`flush()` replays the log on the device in one launch (nkv_pool_apply).  The
device tables then feed the packers directly
(DevicePacker.pack_decode_pool / pack_prefill_pool), so per step only the op
log (a few ints per call) travels to the device, never the block lists.  The
prefix-hash chain stays with the caller, which passes each allocation's
cached-prefix block ids.
"""
from __future__ import annotations

import ctypes
from typing import Iterable

import numpy as np
import torch

from nanokv import _lib
from nanokv.paged_kv.ops import current_stream_handle


class DeviceBlockPool:
    """`num_blocks` blocks of `block_size` tokens, block tables for
    `max_seqs` sequence slots of up to `max_blocks_per_seq` blocks.  The
    state lives in one device buffer owned by this object."""

    def __init__(self, num_blocks: int, block_size: int, *, max_seqs: int,
                 max_blocks_per_seq: int, device: torch.device | str) -> None:
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("DeviceBlockPool requires a ROCm (cuda) device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        lib = _lib.load_library()
        nbytes = int(lib.nkv_pool_bytes(num_blocks, max_seqs, max_blocks_per_seq))
        if nbytes <= 0:
            raise ValueError(
                "need 0 < num_blocks, 0 < max_seqs and 0 < max_blocks_per_seq <= num_blocks "
                "(within the library's limits)"
            )
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self.max_seqs = int(max_seqs)
        self.width = int(max_blocks_per_seq)
        self.memory = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        offsets = (ctypes.c_int64 * 6)()
        _lib.check(lib.nkv_pool_offsets(num_blocks, max_seqs, max_blocks_per_seq, offsets),
                   "nkv_pool_offsets")
        o = list(offsets)
        nb, s, w = self.num_blocks, self.max_seqs, self.width
        self.meta = self.memory[o[0]:o[0] + 64].view(torch.int64)
        self.ring = self.memory[o[1]:o[1] + 8 * nb].view(torch.int32)
        self.qpos = self.memory[o[2]:o[2] + 8 * nb].view(torch.int64)
        self.ref = self.memory[o[3]:o[3] + 4 * nb].view(torch.int32)
        self.tables = self.memory[o[4]:o[4] + 4 * s * w].view(torch.int32).view(s, w)
        self.nblk = self.memory[o[5]:o[5] + 4 * s].view(torch.int32)
        self._desc = _lib.PoolDesc(self.memory.data_ptr(), nb, s, w)
        self._ops: list[tuple[int, int, int, int]] = []
        self._args: list[int] = []
        self._run: set[int] = set()
        self._staging: torch.Tensor | None = None
        self._uploaded: torch.cuda.Event | None = None
        self.reset()

    # -------------------------------------------------------------- control
    def _stream(self) -> int:
        return current_stream_handle(self.device)

    @property
    def desc(self) -> _lib.PoolDesc:
        return self._desc

    def reset(self) -> None:
        """Every block free in id order, every table empty, no error; drops
        the unflushed log."""
        self._ops.clear()
        self._args.clear()
        self._run.clear()
        _lib.check(_lib.load_library().nkv_pool_init(ctypes.byref(self._desc), self._stream()),
                   "nkv_pool_init")

    def _check_slot(self, slot: int) -> int:
        slot = int(slot)
        if not 0 <= slot < self.max_seqs:
            raise ValueError(f"slot {slot} outside [0, {self.max_seqs})")
        return slot

    # ---------------------------------------------- the BlockManager calls
    def allocate(self, slot: int, num_blocks: int, cached: Iterable[int] = ()) -> None:
        """BlockManager.allocate (block_manager.py:185-214) for the sequence
        in `slot`, whose `num_blocks` blocks start with the cached-prefix
        ids that can_allocate found."""
        slot = self._check_slot(slot)
        cached = [int(b) for b in cached]
        if not 0 <= len(cached) <= num_blocks <= self.width:
            raise ValueError("need len(cached) <= num_blocks <= max_blocks_per_seq")
        if len(set(cached)) != len(cached) or any(not 0 <= b < self.num_blocks for b in cached):
            raise ValueError("cached block ids must be distinct and inside the pool")
        self._run.clear()
        self._ops.append((_lib.NKV_POOL_OP_ALLOCATE, slot, int(num_blocks), len(self._args)))
        self._args.append(len(cached))
        self._args.extend(cached)

    def deallocate(self, slot: int) -> None:
        """BlockManager.deallocate (block_manager.py:216-227)."""
        slot = self._check_slot(slot)
        self._run.clear()
        self._ops.append((_lib.NKV_POOL_OP_DEALLOCATE, slot, 0, 0))

    def append(self, slot: int) -> None:
        """One more block for `slot` (BlockManager.may_append when it
        allocates)."""
        slot = self._check_slot(slot)
        if slot in self._run:  # a run of appends must name distinct slots
            self._ops.append((_lib.NKV_POOL_OP_FENCE, 0, 0, 0))
            self._run.clear()
        self._run.add(slot)
        self._ops.append((_lib.NKV_POOL_OP_APPEND, slot, 0, 0))

    def may_append(self, slot: int, seq_len: int) -> bool:
        """block_manager.py:233-236: a new block when the sequence's next
        token opens one (len(seq) % block_size == 1)."""
        if int(seq_len) % self.block_size == 1:
            self.append(slot)
            return True
        return False

    @property
    def pending_ops(self) -> int:
        return len(self._ops)

    def flush(self, timer=None) -> None:
        """Replay the recorded calls on the device (current stream), in
        order, and start a new log.  The pinned staging buffer is reused once
        the previous upload has completed.  `timer` (a
        nanokv.benchmark.LaunchTimer) brackets the apply kernel alone."""
        if not self._ops:
            return
        ops = np.asarray(self._ops, dtype=np.int32).reshape(-1)
        args = np.asarray(self._args, dtype=np.int32)
        total = ops.size + max(args.size, 1)
        if self._uploaded is not None:
            self._uploaded.synchronize()
        if self._staging is None or self._staging.numel() < total:
            self._staging = torch.empty(max(total, 4096), dtype=torch.int32, pin_memory=True)
        host = self._staging.numpy()
        host[: ops.size] = ops
        host[ops.size: ops.size + args.size] = args
        device_log = torch.empty(total, dtype=torch.int32, device=self.device)
        device_log.copy_(self._staging[:total], non_blocking=True)
        if self._uploaded is None:
            self._uploaded = torch.cuda.Event()
        self._uploaded.record(torch.cuda.current_stream(self.device))
        started = timer.start() if timer is not None else None
        status = _lib.load_library().nkv_pool_apply(
            ctypes.byref(self._desc), device_log.data_ptr(), len(self._ops),
            device_log[ops.size:].data_ptr(), args.size, self._stream(),
        )
        if timer is not None:
            timer.stop(started)
        _lib.check(status, "nkv_pool_apply")
        self._ops.clear()
        self._args.clear()
        self._run.clear()

    # ---------------------------------------------------------------- reads
    def error(self) -> tuple[int, int, str] | None:
        """(op index, code, meaning) of the first failed op of the logs
        applied so far, or None.  Synchronizes the stream."""
        meta = self.meta.cpu().tolist()
        if meta[4] == 0:
            return None
        return int(meta[3]) - 1, int(meta[4]), _lib.NKV_POOL_ERRORS.get(int(meta[4]), "?")

    def check(self) -> None:
        err = self.error()
        if err is not None:
            raise RuntimeError(f"block pool op {err[0]} failed: {err[2]} (code {err[1]})")

    def snapshot(self) -> dict:
        """Host copy of the state (synchronizes): the free queue in order,
        the reference counts and every non-empty table."""
        meta = self.meta.cpu().tolist()
        head, tail, live = meta[0], meta[1], meta[2]
        ring = self.ring.cpu().numpy()
        cap = ring.size
        positions = np.arange(head, tail, dtype=np.int64) % cap
        queue = [int(b) for b in ring[positions] if b >= 0]
        nblk = self.nblk.cpu().numpy()
        tables = self.tables.cpu().numpy()
        return {
            "queue": queue,
            "live": int(live),
            "ref": self.ref.cpu().tolist(),
            "tables": {s: tables[s, : nblk[s]].tolist() for s in range(self.max_seqs) if nblk[s] > 0},
            "error": None if meta[4] == 0 else (int(meta[3]) - 1, int(meta[4])),
        }
