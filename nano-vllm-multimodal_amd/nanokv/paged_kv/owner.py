"""Native cache owner of the ``hip`` backend: the counterpart of the
reference's ``torch.classes.nanovllm_paged_kv.PagedKVCache``
(csrc/paged_kv/paged_kv.cpp:41-179, bound at :189-197), with the same
methods: ``tensor()``, ``pending_host_copy_count()`` and
``copy_slots_async(host_slots)``.

The cache is one device tensor.  Slot mappings built on the host go to the
device through the library's transfer lane (nkv_transfer_*): a
non-blocking transfer stream whose copy waits for the compute stream's
earlier work (the slot buffer is reused) and which the compute stream waits
for.  The device slot buffer grows when a larger mapping arrives and is
reused otherwise (same data_ptr); each pinned host tensor is kept alive
until its copy has completed.
"""
from __future__ import annotations

import ctypes
from collections import deque
from threading import Lock
from typing import Sequence

import torch

from nanokv import _lib


class HIPPagedKVCache:
    def __init__(self, sizes: Sequence[int], dtype: torch.dtype, device_index: int) -> None:
        if device_index < 0:
            raise ValueError("device index must be non-negative")
        if not sizes or any(int(s) <= 0 for s in sizes):
            raise ValueError("PagedKVCache dimensions must be positive")
        self._device = torch.device("cuda", device_index)
        self._tensor = torch.empty(tuple(int(s) for s in sizes), dtype=dtype, device=self._device)
        library = _lib.load_library()
        lane = ctypes.c_void_p()
        _lib.check(library.nkv_transfer_create(device_index, ctypes.byref(lane)), "nkv_transfer_create")
        self._lane = lane
        self._slot_buffer: torch.Tensor | None = None
        self._pending: deque[tuple[int, torch.Tensor]] = deque()
        self._lock = Lock()

    def tensor(self) -> torch.Tensor:
        return self._tensor

    def _release_completed(self) -> int:
        in_flight = ctypes.c_int64()
        completed = ctypes.c_int64()
        _lib.check(
            _lib.load_library().nkv_transfer_poll(self._lane, ctypes.byref(in_flight), ctypes.byref(completed)),
            "nkv_transfer_poll",
        )
        while self._pending and self._pending[0][0] <= completed.value:
            self._pending.popleft()
        return len(self._pending)

    def pending_host_copy_count(self) -> int:
        """Host tensors still retained (paged_kv.cpp:97-99): completed
        copies are released lazily, at the next copy_slots_async (which
        starts with release_completed_host_copies, paged_kv.cpp:110,156-167)."""
        with self._lock:
            return len(self._pending)

    def copy_slots_async(self, host_slots: torch.Tensor) -> torch.Tensor:
        """paged_kv.cpp:101-149: an int32 device view of ``host_slots``,
        valid on the current stream of the cache's device."""
        if host_slots.device.type != "cpu":
            raise ValueError("slot mapping source must be a CPU tensor")
        if host_slots.dtype != torch.int32:
            raise ValueError("slot mapping source must be int32")
        if host_slots.dim() != 1 or not host_slots.is_contiguous():
            raise ValueError("slot mapping source must be contiguous and one-dimensional")
        with self._lock:
            self._release_completed()
            count = host_slots.numel()
            if count == 0:
                return torch.empty(0, dtype=torch.int32, device=self._device)
            if not host_slots.is_pinned():
                raise ValueError("slot mapping source must use pinned CPU memory")
            if self._slot_buffer is None or self._slot_buffer.numel() < count:
                self._slot_buffer = torch.empty(count, dtype=torch.int32, device=self._device)
            ticket = ctypes.c_int64()
            stream = torch.cuda.current_stream(self._device).cuda_stream
            status = _lib.load_library().nkv_transfer_h2d(
                self._lane, self._slot_buffer.data_ptr(), host_slots.data_ptr(), count * 4, stream,
                ctypes.byref(ticket),
            )
            _lib.check(status, "nkv_transfer_h2d")
            self._pending.append((ticket.value, host_slots))
            return self._slot_buffer[:count]

    def close(self) -> None:
        lane, self._lane = getattr(self, "_lane", None), None
        if lane is not None and lane.value:
            _lib.load_library().nkv_transfer_destroy(lane)
        self._pending.clear()

    def __del__(self) -> None:  # pragma: no cover - interpreter shutdown order varies
        try:
            self.close()
        except Exception:
            pass
