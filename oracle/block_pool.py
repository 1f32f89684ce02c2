"""CPU restatement of the reference BlockManager's block bookkeeping: the
free-block FIFO, the reference counts and the per-sequence block tables
(nanovllm/engine/block_manager.py:87-118, 159-227).

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: only
tests/ use it, to check the device block pool against it.

The prefix-hash chain (compute_hash, hash_to_block_id, cache_key
verification, hash_blocks; block_manager.py:65-85, 229-258) stays with the
caller: allocate() takes the cached-prefix block ids that can_allocate's hash
walk found, exactly the ids BlockManager.allocate re-derives from the hash
map (:185-214).  Sequences are named by integer slots.

How it is pinned (tests/test_block_pool_oracle.py): hand-derived known
answers of the deque semantics, an independent formulation of the free order
(queue_from_history: free blocks ordered by the time of their latest free,
initial blocks first in id order), bookkeeping invariants after random
scheduler-like runs, and planted mistakes that the known answers catch.
"""
from __future__ import annotations

from collections import deque


class BlockPoolOracle:
    """BlockManager's allocation state without the hash map."""

    def __init__(self, num_blocks: int, width: int | None = None):
        # block_manager.py:51-63: every block free, in id order; ref 0.
        self.num_blocks = num_blocks
        self.width = width
        self.free: deque[int] = deque(range(num_blocks))
        self.ref = [0] * num_blocks
        self.tables: dict[int, list[int]] = {}

    # -- block_manager.py:87-118
    def _allocate_block(self) -> int:
        block_id = self.free.popleft()
        assert self.ref[block_id] == 0
        self.ref[block_id] = 1  # Block.reset(): ref_count = 1
        return block_id

    def _deallocate_block(self, block_id: int) -> None:
        assert self.ref[block_id] == 0
        self.free.append(block_id)

    # -- block_manager.py:185-214
    def allocate(self, slot: int, num_blocks: int, cached: list[int] = ()) -> list[int]:
        """Sequence `slot` takes `num_blocks` blocks: first the cached prefix
        blocks (a used block gains a reference; a free one leaves the free
        queue wherever it stands), then fresh blocks from the queue front."""
        assert not self.tables.get(slot), "allocate on a sequence that holds blocks"
        assert len(cached) <= num_blocks
        if self.width is not None:
            assert num_blocks <= self.width
        table = []
        for block_id in cached:
            if self.ref[block_id] > 0:  # block_id in used_block_ids
                self.ref[block_id] += 1
            else:
                self.ref[block_id] = 1
                self.free.remove(block_id)
            table.append(block_id)
        for _ in range(len(cached), num_blocks):
            table.append(self._allocate_block())
        self.tables[slot] = table
        return list(table)

    # -- block_manager.py:216-227
    def deallocate(self, slot: int) -> None:
        for block_id in reversed(self.tables.get(slot, [])):
            self.ref[block_id] -= 1
            if self.ref[block_id] == 0:
                self._deallocate_block(block_id)
        self.tables[slot] = []

    # -- block_manager.py:233-236 (called when len(seq) % block_size == 1)
    def append(self, slot: int) -> int:
        table = self.tables.setdefault(slot, [])
        if self.width is not None:
            assert len(table) < self.width
        block_id = self._allocate_block()
        table.append(block_id)
        return block_id

    # -- views
    def queue(self) -> list[int]:
        return list(self.free)

    def num_free(self) -> int:
        return len(self.free)

    def table(self, slot: int) -> list[int]:
        return list(self.tables.get(slot, []))


def queue_from_history(num_blocks: int, events) -> list[int]:
    """The free order formulated independently of the deque: `events` is
    the ordered list of ("take", block) and ("free", block) events (a take
    is any block leaving the free set: a pop from the front or a prefix hit
    on a free block; a free is a reference count reaching zero).  Free
    blocks are ordered by the time of their latest free, with never-taken
    blocks first in id order."""
    stamp = {b: (0, b) for b in range(num_blocks)}
    free = set(range(num_blocks))
    for t, (kind, block) in enumerate(events, start=1):
        if kind == "take":
            free.discard(block)
        else:
            free.add(block)
            stamp[block] = (t, 0)
    return sorted(free, key=lambda b: stamp[b])
