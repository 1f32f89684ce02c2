"""Pins the block-pool oracle (oracle.block_pool.BlockPoolOracle, the
restatement of nanovllm/engine/block_manager.py:87-118, 159-227) on the CPU:

  * known answers derived by hand from the reference's deque semantics:
    fresh blocks from the front, frees appended in reversed table order,
    shared prefix blocks freed only by their last holder, a prefix hit on a
    free block removing it from the middle of the queue;
  * an independent formulation of the free order (queue_from_history), fed
    with take/free events derived from the tables alone, after every op of
    seeded scheduler-like runs;
  * bookkeeping invariants after every op;
  * planted mistakes (forward-order frees, a hit block left in the queue,
    frees pushed to the front) that the known answers catch.
"""
from __future__ import annotations

import random
from collections import Counter

import pytest

from oracle.block_pool import BlockPoolOracle, queue_from_history


def test_known_answer_fifo_and_reversed_frees():
    p = BlockPoolOracle(8)
    assert p.allocate(0, 3) == [0, 1, 2]
    assert p.allocate(1, 2) == [3, 4]
    assert p.queue() == [5, 6, 7]
    p.deallocate(0)
    assert p.queue() == [5, 6, 7, 2, 1, 0]
    assert p.allocate(2, 4) == [5, 6, 7, 2]
    assert p.queue() == [1, 0]
    assert p.append(1) == 1
    assert p.table(1) == [3, 4, 1]


def test_known_answer_shared_prefix_and_middle_removal():
    p = BlockPoolOracle(6)
    assert p.allocate(0, 3) == [0, 1, 2]
    assert p.allocate(1, 3, cached=[0, 1]) == [0, 1, 3]
    assert p.ref[:4] == [2, 2, 1, 1]
    p.deallocate(0)                      # only block 2 reaches zero
    assert p.queue() == [4, 5, 2]
    p.deallocate(1)                      # reversed: 3, 1, 0 all reach zero
    assert p.queue() == [4, 5, 2, 3, 1, 0]
    assert p.allocate(2, 2, cached=[1]) == [1, 4]   # 1 leaves the middle
    assert p.queue() == [5, 2, 3, 0]
    assert p.allocate(3, 3, cached=[1, 4]) == [1, 4, 5]  # used blocks gain a ref
    assert p.ref[1] == 2 and p.ref[4] == 2 and p.ref[5] == 1
    assert p.queue() == [2, 3, 0]


class _ForwardFrees(BlockPoolOracle):
    def deallocate(self, slot):
        for b in self.tables.get(slot, []):
            self.ref[b] -= 1
            if self.ref[b] == 0:
                self.free.append(b)
        self.tables[slot] = []


class _HitStaysQueued(BlockPoolOracle):
    def allocate(self, slot, num_blocks, cached=()):
        table = []
        for b in cached:
            self.ref[b] += 1
            table.append(b)
        for _ in range(len(cached), num_blocks):
            table.append(self._allocate_block())
        self.tables[slot] = table
        return table


class _FreesToFront(BlockPoolOracle):
    def _deallocate_block(self, block_id):
        self.free.appendleft(block_id)


@pytest.mark.parametrize("broken", [_ForwardFrees, _HitStaysQueued, _FreesToFront])
def test_planted_mistakes_fail_the_known_answers(broken):
    failed = False
    try:
        p = broken(6)
        p.allocate(0, 3)
        p.allocate(1, 3, cached=[0, 1])
        p.deallocate(0)
        p.deallocate(1)
        assert p.queue() == [4, 5, 2, 3, 1, 0]
        assert p.allocate(2, 2, cached=[1]) == [1, 4]
        assert p.queue() == [5, 2, 3, 0]
    except (AssertionError, ValueError):
        failed = True
    assert failed


def scheduler_like_run(seed: int, num_blocks: int, steps: int, width: int = 64):
    """Yields (op, slot, args) in a scheduler's call order: admissions with
    prefix hits on used and on free (previously released) blocks, decode
    appends, preemptions and finishes."""
    rng = random.Random(seed)
    live: dict[int, int] = {}          # slot -> blocks held
    released: list[list[int]] = []     # tables of finished sequences (hit sources)
    tables: dict[int, list[int]] = {}
    next_slot = 0
    free = num_blocks
    for _ in range(steps):
        kind = rng.random()
        if kind < 0.35 or not live:
            n = rng.randint(1, min(width, 12))
            cached: list[int] = []
            if rng.random() < 0.5:
                source = None
                if live and rng.random() < 0.5:
                    source = tables[rng.choice(list(live))]
                elif released:
                    source = rng.choice(released)
                if source:
                    k = rng.randint(0, min(len(source), n))
                    cached = list(source[:k])
            yield "allocate", next_slot, (n, cached)
            next_slot += 1
        elif kind < 0.75:
            slot = rng.choice(list(live))
            yield "append", slot, ()
        else:
            slot = rng.choice(list(live))
            yield "deallocate", slot, ()
        # the caller reports the new state back through `sync`
        tables, live, released, free = (yield)


def drive(pool_factory, seed, num_blocks=48, steps=300, check=None):
    """Runs a scheduler-like sequence against a pool object with the
    oracle's interface, skipping ops the pool cannot satisfy (the reference
    scheduler asks can_allocate / can_append first)."""
    pool = pool_factory(num_blocks)
    gen = scheduler_like_run(seed, num_blocks, steps)
    tables: dict[int, list[int]] = {}
    released: list[list[int]] = []
    op = next(gen)
    history = []
    while True:
        kind, slot, args = op
        if kind == "allocate":
            n, cached = args
            cached = [b for b in dict.fromkeys(cached)]
            hits_free = sum(1 for b in cached if pool.ref[b] == 0)
            if pool.num_free() - hits_free >= n - len(cached):
                before = Counter(b for t in tables.values() for b in t)
                table = pool.allocate(slot, n, cached)
                tables[slot] = table
                for b in table:
                    if before[b] == 0:
                        history.append(("take", b))
        elif kind == "append":
            if pool.num_free() >= 1 and len(tables[slot]) < 64:
                b = pool.append(slot)
                tables[slot].append(b)
                history.append(("take", b))
        else:
            counts = Counter(b for t in tables.values() for b in t)
            for b in reversed(tables[slot]):
                counts[b] -= 1
                if counts[b] == 0:
                    history.append(("free", b))
            released.append(tables.pop(slot))
            pool.deallocate(slot)
        if check is not None:
            check(pool, tables, history)
        next(gen)
        try:
            op = gen.send((tables, {s: len(t) for s, t in tables.items()}, released, pool.num_free()))
        except StopIteration:
            break
    return pool, tables, history


@pytest.mark.parametrize("seed", range(6))
def test_free_order_matches_history_and_invariants(seed):
    def check(pool, tables, history):
        assert pool.queue() == queue_from_history(pool.num_blocks, history)
        counts = Counter(b for t in tables.values() for b in t)
        for b in range(pool.num_blocks):
            assert pool.ref[b] == counts[b]
        q = pool.queue()
        assert len(q) == len(set(q))
        assert set(q) == {b for b in range(pool.num_blocks) if counts[b] == 0}
        for slot, t in tables.items():
            assert pool.table(slot) == t
            assert len(t) == len(set(t))

    drive(BlockPoolOracle, seed, check=check)
