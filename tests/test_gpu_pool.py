"""Device block pool (nkv_pool_*) vs the block-pool oracle
(oracle.block_pool.BlockPoolOracle, the restatement of
nanovllm/engine/block_manager.py:87-118, 185-236), and packing from the
pool's tables vs packing from the same tables uploaded as CSR.

Every comparison is exact: the free queue in order, every reference count,
every table, and the packed metadata word for word.
"""
from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle.block_pool import BlockPoolOracle

pytestmark = pytest.mark.gpu


def make_pool(device, num_blocks, block_size=16, max_seqs=64, width=None):
    from nanokv.pool import DeviceBlockPool

    return DeviceBlockPool(num_blocks, block_size, max_seqs=max_seqs,
                           max_blocks_per_seq=width or num_blocks, device=device)


def assert_same(pool, oracle, what=""):
    snap = pool.snapshot()
    assert snap["error"] is None, f"{what}: device error {snap['error']}"
    assert snap["queue"] == oracle.queue(), f"{what}: free queue differs"
    assert snap["live"] == oracle.num_free(), f"{what}: free count differs"
    assert snap["ref"] == oracle.ref, f"{what}: reference counts differ"
    expected = {s: t for s, t in oracle.tables.items() if t}
    assert snap["tables"] == expected, f"{what}: tables differ"


def scheduler_steps(seed, num_blocks, steps, max_seqs, width, block_size):
    """Yields lists of ops (one list per scheduler step) that a reference
    scheduler could issue against `oracle` (feasibility checked on it, as
    can_allocate / can_append do): admissions with prefix hits on used and
    on free blocks, decode appends, preemptions and finishes."""
    rng = random.Random(seed)
    oracle = BlockPoolOracle(num_blocks, width)
    lens: dict[int, int] = {}
    released: list[list[int]] = []
    free_slots = list(range(max_seqs))
    for _ in range(steps):
        ops = []
        # admissions
        for _ in range(rng.randint(0, 3)):
            if not free_slots:
                break
            n_tokens = rng.randint(1, block_size * min(width, 10))
            n = -(-n_tokens // block_size)
            cached: list[int] = []
            if rng.random() < 0.6:
                pools = [oracle.table(s) for s in lens] + released[-8:]
                source = rng.choice(pools) if pools else []
                k = rng.randint(0, min(len(source), n - 1)) if n > 1 else 0
                cached = list(dict.fromkeys(source[:k]))
            hits_free = sum(1 for b in cached if oracle.ref[b] == 0)
            if oracle.num_free() - hits_free < n - len(cached):
                continue
            slot = free_slots.pop(rng.randrange(len(free_slots)))
            oracle.allocate(slot, n, cached)
            lens[slot] = n_tokens
            ops.append(("allocate", slot, n, cached))
        # decode: every running sequence grows by one token
        for slot in list(lens):
            if lens[slot] % block_size == 0:          # next token opens a block
                if len(oracle.table(slot)) >= width or oracle.num_free() < 1:
                    released.append(oracle.table(slot))  # preempt
                    oracle.deallocate(slot)
                    ops.append(("deallocate", slot))
                    del lens[slot]
                    free_slots.append(slot)
                    continue
                oracle.append(slot)
                ops.append(("append", slot))
            lens[slot] += 1
        # finishes
        for slot in list(lens):
            if rng.random() < 0.12:
                released.append(oracle.table(slot))
                oracle.deallocate(slot)
                ops.append(("deallocate", slot))
                del lens[slot]
                free_slots.append(slot)
        yield ops, oracle, dict(lens)


def replay(pool, ops):
    for op in ops:
        if op[0] == "allocate":
            pool.allocate(op[1], op[2], op[3])
        elif op[0] == "deallocate":
            pool.deallocate(op[1])
        else:
            pool.append(op[1])
    pool.flush()


@pytest.mark.parametrize("seed,num_blocks,width", [(1, 40, 16), (2, 64, 32), (3, 200, 24), (4, 1500, 64)])
def test_scheduler_runs_match_oracle(gpu_device, seed, num_blocks, width):
    pool = make_pool(gpu_device, num_blocks, max_seqs=48, width=width)
    for step, (ops, oracle, _) in enumerate(scheduler_steps(seed, num_blocks, 120, 48, width, 16)):
        replay(pool, ops)
        assert_same(pool, oracle, f"seed {seed} step {step}")


def test_tombstones_and_compaction(gpu_device):
    """Prefix hits on free blocks leave tombstones; re-freeing those blocks
    grows the ring past num_blocks until a push compacts it."""
    nb = 16
    pool = make_pool(gpu_device, nb, max_seqs=8, width=nb)
    oracle = BlockPoolOracle(nb, nb)
    rng = random.Random(5)
    max_span = 0
    for step in range(200):
        slot = step % 8
        if oracle.table(slot):
            oracle.deallocate(slot)
            pool.deallocate(slot)
        free = oracle.queue()
        back = free[len(free) // 2:]
        if not back:
            continue
        cached = rng.sample(back, rng.randint(1, min(6, len(back))))
        n = len(cached) + rng.randint(0, 2)
        if oracle.num_free() - len(cached) < n - len(cached):
            continue
        oracle.allocate(slot, n, cached)
        pool.allocate(slot, n, cached)
        pool.flush()
        meta = pool.meta.cpu().tolist()
        max_span = max(max_span, meta[1] - meta[0])
        assert meta[1] - meta[0] <= 2 * nb
        assert_same(pool, oracle, f"step {step}")
    assert max_span > nb, "the run never left tombstones in the ring"


def test_pack_from_pool_equals_csr_packing(gpu_device):
    from nanokv.packing import DevicePacker, SequenceBatch

    bs = 16
    packer = DevicePacker(gpu_device, bs)
    pool = make_pool(gpu_device, 600, block_size=bs, max_seqs=48, width=40)
    steps = scheduler_steps(9, 600, 60, 48, 40, bs)
    for step, (ops, oracle, lens) in enumerate(steps):
        replay(pool, ops)
        if not lens:
            continue
        slots = sorted(lens)
        tokens = np.array([lens[s] for s in slots], dtype=np.int32)  # tables cover ceil(len/bs)
        tables = [oracle.table(s) for s in slots]
        batch = SequenceBatch.from_block_lists(tokens, tables)
        a = packer.pack_decode(batch)
        b = packer.pack_decode_pool(pool, slots, tokens)
        for name in ("slot_mapping", "context_lens", "cu_seqlens_k", "block_tables"):
            assert torch.equal(getattr(a, name), getattr(b, name)), f"step {step}: {name}"
        # prefill view of the same tables: a chunk of each sequence scheduled
        cached = np.array([max(0, int(t) - 1 - (step % 5)) for t in tokens], dtype=np.int32)
        sched = tokens - cached
        pbatch = SequenceBatch.from_block_lists(tokens, tables, num_cached_tokens=cached,
                                                num_scheduled_tokens=sched, num_prompt_tokens=tokens)
        pa = packer.pack_prefill(pbatch, force_block_tables=True)
        pb = packer.pack_prefill_pool(pool, slots, cached, sched, tokens, force_block_tables=True)
        for name in ("cu_seqlens_q", "cu_seqlens_k", "slot_mapping", "block_tables",
                     "full_context_lens", "query_start_lens"):
            assert torch.equal(getattr(pa, name), getattr(pb, name)), f"step {step}: prefill {name}"


def test_invalid_ops_stop_the_log_and_keep_the_state(gpu_device):
    """Each invalid op alone in a log: the error is recorded with its code
    and the state is untouched.  Ops the Python recorder refuses are written
    into the raw log to reach the device's own checks."""
    pool = make_pool(gpu_device, 8, max_seqs=4, width=4)
    oracle = BlockPoolOracle(8, 4)

    def setup():
        pool.reset()
        pool.allocate(0, 3)
        pool.flush()
        assert_same(pool, oracle, "setup")

    oracle.allocate(0, 3)

    def raw(op, args=()):
        pool._ops.append(op)
        pool._args.extend(args)

    def two_allocations():  # 5 free: the first takes 4, the second finds 1
        pool.allocate(1, 4)
        pool.allocate(2, 4)

    cases = [
        (3, lambda: pool.allocate(0, 1)),                          # slot 0 holds blocks
        (5, two_allocations),                                      # valid prefix, then stop
        (2, lambda: raw((3, 9, 0, 0))),                            # slot outside the pool
        (1, lambda: raw((9, 0, 0, 0))),                            # unknown op
        (6, lambda: raw((1, 1, 2, len(pool._args)), [1, 99])),     # cached id outside
        (7, lambda: raw((1, 1, 2, 1000))),                         # args offset outside
        (7, lambda: raw((1, 1, 2, len(pool._args)), [3, 4, 5, 6])),  # 3 cached > 2 blocks
    ]
    for code, record in cases:
        setup()
        before = pool.snapshot()
        record()
        pool.flush()
        err = pool.error()
        assert err is not None and err[1] == code, (code, err)
        after = pool.snapshot()
        if code == 5:
            # the valid prefix (the first allocate) is applied, then the log stops
            o = BlockPoolOracle(8, 4)
            o.allocate(0, 3)
            o.allocate(1, 4)
            assert after["queue"] == o.queue() and after["tables"] == {0: [0, 1, 2], 1: [3, 4, 5, 6]}
            continue
        for key in ("queue", "live", "ref", "tables"):
            assert after[key] == before[key], (code, key)

    # append past the table width, alone in its log
    setup()
    pool.append(0)
    pool.flush()
    assert pool.error() is None
    before = pool.snapshot()
    pool.append(0)
    pool.flush()
    assert pool.error()[1] == 4
    assert pool.snapshot()["tables"] == before["tables"]
    # a log after a failed one is ignored until reset
    pool.append(1)
    pool.flush()
    assert pool.snapshot()["tables"] == before["tables"]
    pool.reset()
    assert pool.error() is None


def sequential(oracle, ops, width, max_seqs):
    """The op log one op at a time on the oracle, stopping at the first
    invalid op: returns (index, code) of that op, or None."""
    for idx, op in enumerate(ops):
        kind, slot = op[0], op[1]
        if kind == "fence":
            continue
        if not 0 <= slot < max_seqs:
            return idx, 2
        if kind == "allocate":
            n, cached = op[2], op[3]
            if oracle.table(slot):
                return idx, 3
            if not 0 <= n <= width or len(cached) > n:
                return idx, 7
            hits_free = sum(1 for b in cached if oracle.ref[b] == 0)
            if oracle.num_free() - hits_free < n - len(cached):
                return idx, 5
            oracle.allocate(slot, n, cached)
        elif kind == "append":
            if len(oracle.table(slot)) >= width:
                return idx, 4
            if oracle.num_free() < 1:
                return idx, 5
            oracle.append(slot)
        else:
            oracle.deallocate(slot)
    return None


def raw_log(pool, ops):
    """Writes ops straight into the pool's log (no recorder checks, no
    fences), as a C caller could."""
    from nanokv import _lib

    codes = {"allocate": _lib.NKV_POOL_OP_ALLOCATE, "deallocate": _lib.NKV_POOL_OP_DEALLOCATE,
             "append": _lib.NKV_POOL_OP_APPEND, "fence": _lib.NKV_POOL_OP_FENCE}
    for op in ops:
        if op[0] == "allocate":
            pool._ops.append((codes["allocate"], op[1], op[2], len(pool._args)))
            pool._args.extend([len(op[3]), *op[3]])
        else:
            pool._ops.append((codes[op[0]], op[1], 0, 0))


@pytest.mark.parametrize("case", [
    # appends repeating a slot inside one run
    [("append", 0), ("append", 1), ("append", 0), ("append", 2), ("append", 0), ("append", 1)],
    # allocations without cached ids repeating a slot (the repeat is busy)
    [("allocate", 4, 2, []), ("allocate", 5, 1, []), ("allocate", 4, 1, []), ("allocate", 6, 1, [])],
    # a bad slot in the middle of an append run
    [("append", 0), ("append", 1), ("append", 11), ("append", 2)],
    # an append past the table width in the middle of a run
    [("append", 3), ("append", 3), ("append", 3), ("append", 3), ("append", 3), ("append", 1)],
    # more appends than free blocks
    [("append", s % 4) for s in range(40)],
    # allocations whose running total passes the free count
    [("allocate", 4, 3, []), ("allocate", 5, 4, []), ("allocate", 6, 4, []), ("allocate", 7, 1, [])],
    # bad sizes inside an allocation run
    [("allocate", 4, 2, []), ("allocate", 5, 9, []), ("allocate", 6, 1, [])],
    # runs split by other ops
    [("allocate", 4, 1, []), ("append", 4), ("deallocate", 0), ("allocate", 0, 2, []),
     ("append", 0), ("fence", 0), ("append", 0), ("allocate", 5, 1, [4])],
    # a deallocation run (no sharing), with a repeat and an empty slot
    [("append", 1), ("deallocate", 0), ("deallocate", 1), ("deallocate", 0), ("deallocate", 6),
     ("deallocate", 2)],
    # a deallocation run over a shared block (one-op path), then a bad slot
    [("allocate", 4, 2, [1]), ("allocate", 5, 3, [1, 0]), ("deallocate", 1), ("deallocate", 4),
     ("deallocate", 0), ("deallocate", 5), ("deallocate", 9)],
])
def test_runs_match_one_op_at_a_time(gpu_device, case):
    width, max_seqs, nb = 5, 8, 14
    pool = make_pool(gpu_device, nb, max_seqs=max_seqs, width=width)
    oracle = BlockPoolOracle(nb, width)
    for s in range(4):  # slots 0..3 hold one block each; 10 free
        pool.allocate(s, 1)
        oracle.allocate(s, 1)
    pool.flush()
    assert_same(pool, oracle, "setup")
    expected_err = sequential(oracle, case, width, max_seqs)
    raw_log(pool, case)
    pool.flush()
    snap = pool.snapshot()
    assert snap["error"] == expected_err
    assert snap["queue"] == oracle.queue()
    assert snap["ref"] == oracle.ref
    assert snap["tables"] == {s: t for s, t in oracle.tables.items() if t}


def test_host_side_checks(gpu_device):
    pool = make_pool(gpu_device, 8, max_seqs=4, width=4)
    with pytest.raises(ValueError):
        pool.allocate(4, 1)
    with pytest.raises(ValueError):
        pool.allocate(0, 2, [1, 1])
    with pytest.raises(ValueError):
        pool.allocate(0, 5)
    with pytest.raises(ValueError):
        make_pool(gpu_device, 0)
    assert pool.may_append(0, 17) is True and pool.may_append(1, 18) is False
    assert pool.pending_ops == 1


def test_decode_step_scale(gpu_device):
    """The 256-sequence decode step's block lists (contexts up to 16384
    tokens, 256-token blocks) built by admissions, then 300 decode steps of
    appends with churn, against the oracle."""
    from nanokv import workloads

    wl = workloads.build("decode_step", num_layers=1)
    bs, nb = wl.block_size, wl.num_blocks
    pool = make_pool(gpu_device, nb, block_size=bs, max_seqs=512, width=80)
    oracle = BlockPoolOracle(nb, 80)
    lens = {}
    for slot, n_tokens in enumerate(wl.num_tokens.tolist()):
        n = -(-n_tokens // bs)
        oracle.allocate(slot, n)
        pool.allocate(slot, n)
        lens[slot] = n_tokens
    pool.flush()
    assert_same(pool, oracle, "admissions")
    rng = random.Random(3)
    next_slot = len(lens)
    for step in range(300):
        for slot in list(lens):
            if lens[slot] % bs == 0:
                if oracle.num_free() < 1 or len(oracle.table(slot)) >= 80:
                    continue
                oracle.append(slot)
                pool.append(slot)
            lens[slot] += 1
        for slot in rng.sample(list(lens), 2):
            oracle.deallocate(slot)
            pool.deallocate(slot)
            del lens[slot]
            n_tokens = rng.randint(256, 4096)
            n = -(-n_tokens // bs)
            if oracle.num_free() >= n:
                slot = next_slot % 512
                next_slot += 1
                if slot in lens or oracle.table(slot):
                    continue
                oracle.allocate(slot, n)
                pool.allocate(slot, n)
                lens[slot] = n_tokens
        pool.flush()
        if step % 50 == 49:
            assert_same(pool, oracle, f"step {step}")
    assert_same(pool, oracle, "end")
