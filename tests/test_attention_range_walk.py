"""The range decode kernel's per-wavefront control flow, checked on the CPU.

attn_decode_range_kernel (csrc/nkv_attention.hip) runs each worker's range
as two walkers over one ring of S chunk buffers: the copy walker issues
chunk j + S - 1 while the compute walker computes chunk j, and the next
sequence's block ids and q are copied into LDS ahead of time.  No barrier
or fence orders any of it: every read of an LDS buffer is ordered after the
copy that fills it by a counted wait on the vector-memory counter
(s_waitcnt vmcnt(n): "at most n of my loads still outstanding", loads
completing in issue order).

This test restates that control flow step for step, with the counter as an
in-order queue, over plans restated from the lengths (the plan kernel's own
output is compared with the same restatement on the GPU), and asserts:
  * a chunk is computed only after its 8 copies have left the queue, with
    its own sequence's q, each chunk of each context exactly once;
  * the id and q buffers are read only after their copies have landed and
    are never refilled before they were read;
  * every partial a worker writes lies in its sequence's first_part range.
Two planted mistakes (dropping the wait before reading a late q, or the
wait before reading the prefetched block ids) must be caught.
"""
from __future__ import annotations

import random

import pytest

from test_gpu_attention import KEYS, expected_attention_plan

COPIES = 8  # copy instructions per chunk (K and V, 16 keys)


class Hazard(AssertionError):
    pass


def run_worker(p, w, group, slots, *, late_q_wait=True, id_wait=True):
    """Walk worker w of plan p as the kernel does; returns {(seq, chunk)}."""
    workers, units, n, _ = p["header"]
    lens, vstart, first = p["lens"], p["vstart"], p["first"]
    s0, c0, end = (int(x) for x in p["records"][w][:3])
    computed = []
    if lens[s0] <= 0 or vstart[s0] + c0 >= end:
        return computed
    queue, landed = [], set()
    counter = [0]

    def tag(kind, info):
        counter[0] += 1
        return (kind, info, counter[0])

    def wait(outstanding):
        while len(queue) > outstanding:
            landed.add(queue.pop(0))

    buffers = {"ids": None, "q": None}

    def next_seq(s):
        for t in range(s + 1, n):
            if lens[t] > 0:
                return t if vstart[t] < end else -1
        return -1

    def prefetch(kind, s, count):
        b = buffers[kind]
        if b is not None and not b[2]:
            raise Hazard(f"{kind} buffer refilled before it was read")
        tags = [tag(kind, s) for _ in range(count)]
        queue.extend(tags)
        buffers[kind] = [tags, s, False]

    def read(kind, s):
        b = buffers[kind]
        if b is None or b[1] != s:
            raise Hazard(f"{kind} buffer holds another sequence")
        if not all(t in landed for t in b[0]):
            raise Hazard(f"{kind} buffer read before its copy landed")
        b[2] = True

    ring = [None] * slots

    def issue(slot, s, c):
        if ring[slot] is not None:
            raise Hazard("ring slot refilled before its chunk was computed")
        tags = [tag("chunk", (s, c)) for _ in range(COPIES)]
        queue.extend(tags)
        ring[slot] = (s, c, tags)

    q_copies = (group * 256 + 1023) // 1024
    q_in_lds = group <= 8
    cw = {"s": s0, "c": c0, "len": int(lens[s0]), "next": next_seq(s0)}

    def step():  # the copy walker's step()
        cw["c"] += 1
        if cw["c"] * KEYS < cw["len"]:
            return vstart[cw["s"]] + cw["c"] < end
        if cw["next"] < 0:
            return False
        if id_wait:
            wait(COPIES)
        cw["s"], cw["c"], cw["len"] = cw["next"], 0, int(lens[cw["next"]])
        read("ids", cw["s"])
        cw["next"] = next_seq(cw["s"])
        if cw["next"] >= 0:
            prefetch("ids", cw["next"], 1)
        return True

    # prologue: plain loads of the first ids and q, waited for
    q_held = s0
    wait(0)
    part = int(first[s0]) + (w - ((int(vstart[s0]) + 1) * workers - 1) // units)
    cs, cc, clen = s0, c0, int(lens[s0])
    q_stale = q_late = False
    if cw["next"] >= 0:
        prefetch("ids", cw["next"], 1)
        if q_in_lds:
            prefetch("q", cw["next"], q_copies)
    issue(0, cw["s"], cw["c"])
    issued, copying = 1, True
    for k in range(1, slots - 1):
        if copying and step():
            issue(k, cw["s"], cw["c"])
            issued += 1
        else:
            copying = False
    slot, slot_in, j = 0, issued % slots, 0
    while True:
        if copying and step():
            issue(slot_in, cw["s"], cw["c"])
            issued += 1
            slot_in = (slot_in + 1) % slots
        else:
            copying = False
        wait(COPIES * min(issued - 1 - j, 3))
        if q_stale:
            if q_in_lds:
                if q_late and late_q_wait:
                    wait(0)
                read("q", cs)
                after = next_seq(cs)
                if after >= 0:
                    prefetch("q", after, q_copies)
                    q_late = after <= cw["s"]
            else:
                wait(0)  # plain loads of q, waited for
            q_held = cs
            q_stale = False
        s, c, tags = ring[slot]
        if not all(t in landed for t in tags):
            raise Hazard("chunk computed before its copies landed")
        if (s, c) != (cs, cc) or q_held != cs:
            raise Hazard("chunk computed out of step or with another sequence's q")
        computed.append((s, c))
        ring[slot] = None
        last = j + 1 == issued
        cc += 1
        if last or cc * KEYS >= clen:
            if not first[cs] <= part < first[cs + 1]:
                raise Hazard(f"partial {part} outside sequence {cs}'s range")
            if last:
                break
            cs = next_seq(cs)
            cc, clen, part, q_stale = 0, int(lens[cs]), int(first[cs]), True
        slot = (slot + 1) % slots
        j += 1
    return computed


def run_plan(lens, group, hkv, slots, **rules):
    p = expected_attention_plan(lens, hkv)
    done = []
    for w in range(p["header"][0]):
        done += run_worker(p, w, group, slots, **rules)
    want = [(i, c) for i, n in enumerate(lens) for c in range(-(-n // KEYS))]
    assert sorted(done) == want, "a chunk computed twice or never"


def random_lengths(rng, kind):
    if kind == 0:  # many short contexts, one-chunk sequences inside ranges
        return [rng.choice([0, 0, 1, 5, 16, 17, 31, 33, 48]) for _ in range(rng.randint(1, 3000))]
    if kind == 1:  # long contexts among short ones
        lens = [rng.randint(0, 40) for _ in range(rng.randint(1, 800))]
        for _ in range(rng.randint(0, 8)):
            lens[rng.randrange(len(lens))] = rng.randint(1000, 30000)
        return lens
    if kind == 2:  # the decode step's range of lengths
        return [rng.randint(256, 16384) for _ in range(rng.randint(1, 300))]
    return [rng.randint(0, 200) for _ in range(rng.randint(1, 50))]


@pytest.mark.parametrize("seed", range(8))
def test_range_walk_orders_every_read_after_its_copy(seed):
    rng = random.Random(seed)
    for trial in range(5):
        lens = random_lengths(rng, (seed + trial) % 4) or [1]
        if sum(lens) == 0:
            lens[0] = 1
        run_plan(lens, rng.choice([1, 2, 4, 7, 8, 9, 16]), rng.choice([1, 2, 3, 4]),
                 rng.choice([2, 3, 4]))


@pytest.mark.parametrize("rule", ["late_q_wait", "id_wait"])
def test_planted_missing_waits_are_caught(rule):
    """Without the wait before reading a q copied after its sequence's first
    chunk, or before reading the prefetched block ids, some plan of short
    sequences reads a buffer too early."""
    rng = random.Random(11)
    with pytest.raises(Hazard):
        for _ in range(40):
            lens = [rng.choice([1, 5, 16, 17, 33]) for _ in range(rng.randint(200, 2000))]
            run_plan(lens, 8, 2, rng.choice([2, 3]), **{rule: False})
