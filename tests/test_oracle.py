"""Pins the oracle before anything is compared against it.

How each oracle function is pinned:

  store / gather (oracle.paged_kv, oracle.c_oracle)
    * golden vectors re-entered from the reference's tests
      (tests/golden/paged_kv_golden.json, built by explicit placement);
    * torch's own CPU index_copy_ / index_select, the library routines the
      reference's pytorch backend calls (pytorch_backend.py:37-38, 50);
    * row-by-row brute force on tiny inputs;
    * numpy form == C form on random inputs of every dtype width.
  gather_varlen
    * == the concatenation of per-request gathers (attention.py:254-259,
      287-292), and C form == numpy form.
  prepare_decode / prepare_prefill / pack_* (C)
    * hand-derived fixtures (golden "packing" cases);
    * closed-form invariants on random batches: cu_seqlens start at 0 and
      are non-decreasing, cu_seqlens_q[-1] = number of slots, slots unique
      and inside the owning block list, padding -1, decode slot =
      bt[(n-1)//BS]*BS + (n-1)%BS;
    * C form == reference-loop form.
  effective_bytes / linear_percentile
    * the reference's own known answers (test_bench_paged_kv.py:58-89).

A few tests plant a mistake in a copy of an oracle function and check that
the goldens catch it, so a plausible bug (off-by-one row, swapped operands,
dropped skip of slot -1) cannot pass silently.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import paged_kv as ref

GOLDEN = json.loads((Path(__file__).parent / "golden" / "paged_kv_golden.json").read_text())


def _arr(values, dtype=np.float32):
    return np.asarray(values, dtype=dtype)


# ------------------------------------------------------------------ goldens

@pytest.mark.parametrize("case", ["store", "slot_matrix", "native_allocation"])
def test_store_matches_golden(case):
    g = GOLDEN[case]
    dtype = np.int16 if g.get("dtype") == "int16" else np.float32
    key, value = _arr(g["key"], dtype), _arr(g["value"], dtype)
    for impl in ("numpy", "c"):
        kc = np.full(g["cache_shape"], g["cache_fill"], dtype=dtype)
        vc = np.full(g["cache_shape"], g["cache_fill"], dtype=dtype)
        slots = _arr(g["slot_mapping"], np.int32)
        if impl == "numpy":
            ref.store(key, value, kc, vc, slots)
        else:
            c_oracle.store(key, value, kc, vc, slots, threads=2)
        np.testing.assert_array_equal(kc, _arr(g["expected_key_cache"], dtype))
        np.testing.assert_array_equal(vc, _arr(g["expected_value_cache"], dtype))


@pytest.mark.parametrize("case", ["gather", "sdpa_gather"])
def test_gather_matches_golden(case):
    g = GOLDEN[case]
    cache = _arr(g["cache"])
    expected = _arr(g["expected"])
    np.testing.assert_array_equal(ref.gather(cache, g["block_table"], g["sequence_length"]), expected)
    np.testing.assert_array_equal(
        c_oracle.gather(cache, g["block_table"], g["sequence_length"]), expected
    )


@pytest.mark.parametrize("case", ["slot_matrix", "native_allocation"])
def test_gather_after_store_matches_golden(case):
    g = GOLDEN[case]
    dtype = np.int16 if g.get("dtype") == "int16" else np.float32
    cache = _arr(g["expected_key_cache"], dtype)
    expected = _arr(g["expected_gather"], dtype)
    np.testing.assert_array_equal(ref.gather(cache, g["block_table"], g["sequence_length"]), expected)
    np.testing.assert_array_equal(
        c_oracle.gather(cache, g["block_table"], g["sequence_length"], threads=3), expected
    )


def test_decode_replay_golden():
    g = GOLDEN["decode_replay"]
    kc = np.full(g["cache_shape"], g["cache_fill"], dtype=np.float32)
    vc = kc.copy()
    for step in range(g["steps"]):
        key = np.full((1, 1, 64), step, dtype=np.float32)
        ref.store(key, -key, kc, vc, np.array([step % 16], np.int32))
    np.testing.assert_array_equal(kc[0, :, 0, 0], g["expected_key_column"])
    np.testing.assert_array_equal(vc[0, :, 0, 0], g["expected_value_column"])


def _seq_states(case):
    out = []
    for s in case["seqs"]:
        if case.get("decode"):
            out.append(ref.SeqState(num_tokens=s["num_tokens"], block_table=list(s["block_table"])))
        else:
            out.append(ref.SeqState(
                num_tokens=s["num_cached"] + s["num_scheduled"],
                block_table=list(s["block_table"]),
                num_prompt_tokens=s["num_prompt"],
                num_cached_tokens=s["num_cached"],
                num_scheduled_tokens=s["num_scheduled"],
            ))
    return out


@pytest.mark.parametrize("case", GOLDEN["packing"], ids=lambda c: c["name"])
def test_packing_matches_hand_fixtures(case):
    seqs = _seq_states(case)
    bs = case["block_size"]
    offsets, ids = ref.csr(seqs)
    if case.get("decode"):
        got = ref.prepare_decode(seqs, bs)
        width = got["block_tables"].shape[1]
        c_got = c_oracle.pack_decode([s.num_tokens for s in seqs], offsets, ids, bs, width)
        for out in (got, c_got):
            np.testing.assert_array_equal(out["slot_mapping"], case["slot_mapping"])
            np.testing.assert_array_equal(out["context_lens"], case["context_lens"])
            np.testing.assert_array_equal(out["block_tables"], case["block_tables"])
            np.testing.assert_array_equal(out["cu_seqlens_k"], case["cu_seqlens_k"])
        return
    got = ref.prepare_prefill(seqs, bs)
    for key in ("slot_mapping", "cu_seqlens_q", "cu_seqlens_k", "full_context_lens", "query_start_lens"):
        np.testing.assert_array_equal(got[key], case[key], err_msg=key)
    assert got["max_seqlen_q"] == case["max_seqlen_q"]
    assert got["max_seqlen_k"] == case["max_seqlen_k"]
    if case["block_tables"] is None:
        assert got["block_tables"] is None
    else:
        np.testing.assert_array_equal(got["block_tables"], case["block_tables"])
    width = max(len(s.block_table) for s in seqs)
    c_got = c_oracle.pack_prefill(
        [s.num_cached_tokens for s in seqs], [s.num_scheduled_tokens for s in seqs],
        offsets, ids, bs, width,
    )
    np.testing.assert_array_equal(c_got["slot_mapping"], case["slot_mapping"])
    np.testing.assert_array_equal(c_got["cu_seqlens_q"], case["cu_seqlens_q"])
    np.testing.assert_array_equal(c_got["cu_seqlens_k"], case["cu_seqlens_k"])


def test_benchmark_known_answers():
    g = GOLDEN["benchmark"]
    for c in g["effective_bytes"]:
        assert ref.effective_bytes(c["operation"], c["tokens"], c["heads"], c["dim"], c["element_size"]) == c["expected"]
    p = g["percentiles"]
    assert ref.linear_percentile(p["values"], 0.50) == p["p50"]
    assert ref.linear_percentile(p["values"], 0.95) == pytest.approx(p["p95"])
    assert ref.linear_percentile(p["values"], 0.99) == pytest.approx(p["p99"])


# ------------------------------------------------- torch library routines

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("heads,dim", [(1, 64), (2, 128), (8, 80)])
def test_store_and_gather_equal_torch_index_ops(dtype, heads, dim):
    """The reference pytorch backend is index_copy_ / index_select on the
    slot-flattened cache; the oracle must agree bit for bit (compared as
    integer words)."""
    g = torch.Generator().manual_seed(23 + heads + dim)
    nb, bs, t = 41, 16, 257
    key = torch.randn(t, heads, dim, generator=g).to(dtype)
    value = torch.randn(t, heads, dim, generator=g).to(dtype)
    slots = torch.randperm(nb * bs, generator=g)[:t].to(torch.int32)
    slots[::11] = -1
    kc = torch.randn(nb, bs, heads, dim, generator=g).to(dtype)
    vc = torch.randn(nb, bs, heads, dim, generator=g).to(dtype)
    exp_k, exp_v = kc.clone(), vc.clone()
    valid = slots >= 0
    exp_k.flatten(0, 1).index_copy_(0, slots[valid].long(), key[valid])
    exp_v.flatten(0, 1).index_copy_(0, slots[valid].long(), value[valid])

    word = torch.int16 if dtype != torch.float32 else torch.int32
    k_np, v_np = key.view(word).numpy(), value.view(word).numpy()
    got_k, got_v = kc.view(word).numpy().copy(), vc.view(word).numpy().copy()
    ref.store(k_np, v_np, got_k, got_v, slots.numpy())
    np.testing.assert_array_equal(got_k, exp_k.view(word).numpy())
    np.testing.assert_array_equal(got_v, exp_v.view(word).numpy())
    c_k, c_v = kc.view(word).numpy().copy(), vc.view(word).numpy().copy()
    c_oracle.store(k_np, v_np, c_k, c_v, slots.numpy(), threads=4)
    np.testing.assert_array_equal(c_k, got_k)
    np.testing.assert_array_equal(c_v, got_v)

    table = torch.randperm(nb, generator=g).to(torch.int32)
    for length in (0, 1, 15, 16, 17, 300, nb * bs):
        need = -(-length // bs)
        expected = exp_k.index_select(0, table[:need].long()).flatten(0, 1)[:length]
        got = ref.gather(exp_k.view(word).numpy(), table.numpy(), length)
        np.testing.assert_array_equal(got, expected.view(word).numpy())
        got_c = c_oracle.gather(exp_k.view(word).numpy(), table.numpy(), length, threads=2)
        np.testing.assert_array_equal(got_c, got)


def test_store_with_strided_fused_qkv_rows_matches_torch():
    """tests/test_paged_kv_cuda.py:51-78: K and V are views into a packed
    QKV tensor (token stride > heads*dim)."""
    g = torch.Generator().manual_seed(29)
    packed = torch.randn(9, 8, 64, generator=g).to(torch.float16)
    key, value = packed[:, 4:6], packed[:, 6:8]
    assert key.stride(0) > key.shape[1] * key.shape[2]
    slots = torch.tensor([0, 17, 4, 31, 8, 23, 2, 15, 9], dtype=torch.int32)
    exp_k = torch.full((4, 8, 2, 64), -3, dtype=torch.float16)
    exp_v = exp_k.clone()
    exp_k.flatten(0, 1).index_copy_(0, slots.long(), key)
    exp_v.flatten(0, 1).index_copy_(0, slots.long(), value)
    kc = np.full((4, 8, 2, 64), -3, dtype=np.float16).view(np.int16)
    vc = kc.copy()
    c_oracle.store(key.view(torch.int16).numpy(), value.view(torch.int16).numpy(), kc, vc, slots.numpy())
    np.testing.assert_array_equal(kc, exp_k.view(torch.int16).numpy())
    np.testing.assert_array_equal(vc, exp_v.view(torch.int16).numpy())


# --------------------------------------------------------------- brute force

def test_store_and_gather_equal_brute_force():
    rng = np.random.default_rng(5)
    for trial in range(20):
        nb, bs, h, d = rng.integers(1, 6), rng.integers(1, 5), rng.integers(1, 3), rng.integers(1, 5)
        t = int(rng.integers(0, nb * bs + 1))
        key = rng.integers(-1000, 1000, (t, h, d)).astype(np.int16)
        value = rng.integers(-1000, 1000, (t, h, d)).astype(np.int16)
        slots = rng.permutation(nb * bs)[:t].astype(np.int32)
        if t:
            slots[rng.random(t) < 0.3] = -1
        kc = rng.integers(-9, 9, (nb, bs, h, d)).astype(np.int16)
        vc = rng.integers(-9, 9, (nb, bs, h, d)).astype(np.int16)
        bk, bv = kc.copy(), vc.copy()
        ref.store(key, value, kc, vc, slots)
        ref.store_bruteforce(key, value, bk, bv, slots)
        np.testing.assert_array_equal(kc, bk)
        np.testing.assert_array_equal(vc, bv)
        table = rng.permutation(nb).astype(np.int32)
        length = int(rng.integers(0, nb * bs + 1))
        np.testing.assert_array_equal(ref.gather(kc, table, length), ref.gather_bruteforce(kc, table, length))


def test_gather_varlen_is_concatenation_of_gathers():
    rng = np.random.default_rng(9)
    nb, bs = 64, 8
    cache = rng.integers(-30000, 30000, (nb, bs, 2, 16)).astype(np.int16)
    lens = rng.integers(0, 60, 13)
    width = int(max(1, (lens.max() + bs - 1) // bs))
    tables = np.full((13, width), -1, np.int32)
    for i, n in enumerate(lens):
        need = -(-int(n) // bs)
        tables[i, :need] = rng.choice(nb, need, replace=False)
    expected = np.concatenate([ref.gather(cache, tables[i], int(n)) for i, n in enumerate(lens)])
    np.testing.assert_array_equal(ref.gather_varlen(cache, tables, lens), expected)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    np.testing.assert_array_equal(c_oracle.gather_varlen(cache, tables, cu, threads=4), expected)


# ------------------------------------------------------- packing invariants

def _random_batch(rng, b, bs, decode):
    seqs = []
    next_block = 0
    for _ in range(b):
        if decode:
            n = int(rng.integers(1, 50))
            need = -(-n // bs)
            seqs.append(ref.SeqState(num_tokens=n, block_table=list(range(next_block, next_block + need))))
            next_block += need
        else:
            cached = int(rng.integers(0, 3)) * bs if rng.random() < 0.5 else 0
            q = int(rng.integers(1, 40))
            need = -(-(cached + q) // bs)
            table = list(range(next_block, next_block + need)) if rng.random() > 0.1 else []
            next_block += need
            seqs.append(ref.SeqState(cached + q, table, cached + q + int(rng.integers(0, 5)), cached, q))
    perm = rng.permutation(max(next_block, 1))
    for s in seqs:
        s.block_table = [int(perm[x]) for x in s.block_table]
    return seqs


@pytest.mark.parametrize("seed", range(6))
def test_prefill_packing_invariants_and_c_form(seed):
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([4, 16, 256]))
    seqs = _random_batch(rng, int(rng.integers(1, 30)), bs, decode=False)
    got = ref.prepare_prefill(seqs, bs)
    cu_q, cu_k, slots = got["cu_seqlens_q"], got["cu_seqlens_k"], got["slot_mapping"]
    assert cu_q[0] == 0 and cu_k[0] == 0
    assert (np.diff(cu_q) >= 0).all() and (np.diff(cu_k) >= 0).all()
    emitted = sum(s.num_scheduled_tokens for s in seqs if s.block_table)
    assert slots.size == emitted
    assert cu_q[-1] == sum(s.num_scheduled_tokens for s in seqs)
    assert len(np.unique(slots)) == slots.size
    cursor = 0
    for s in seqs:
        if not s.block_table:
            continue
        for p in range(s.num_cached_tokens, s.num_cached_tokens + s.num_scheduled_tokens):
            assert slots[cursor] == s.block_table[p // bs] * bs + p % bs
            assert slots[cursor] // bs in s.block_table
            cursor += 1
    has_cached = any(s.num_cached_tokens > 0 for s in seqs)
    assert (got["block_tables"] is not None) == has_cached
    offsets, ids = ref.csr(seqs)
    width = max(len(s.block_table) for s in seqs)
    c_got = c_oracle.pack_prefill(
        [s.num_cached_tokens for s in seqs], [s.num_scheduled_tokens for s in seqs], offsets, ids, bs, width
    )
    np.testing.assert_array_equal(c_got["slot_mapping"], slots)
    np.testing.assert_array_equal(c_got["cu_seqlens_q"], cu_q)
    np.testing.assert_array_equal(c_got["cu_seqlens_k"], cu_k)
    np.testing.assert_array_equal(c_got["block_tables"], ref.prepare_block_tables(seqs))


@pytest.mark.parametrize("seed", range(6))
def test_decode_packing_invariants_and_c_form(seed):
    rng = np.random.default_rng(100 + seed)
    bs = int(rng.choice([4, 16, 256]))
    seqs = _random_batch(rng, int(rng.integers(1, 40)), bs, decode=True)
    got = ref.prepare_decode(seqs, bs)
    for i, s in enumerate(seqs):
        n = s.num_tokens
        assert got["slot_mapping"][i] == s.block_table[(n - 1) // bs] * bs + (n - 1) % bs
        row = got["block_tables"][i]
        assert list(row[: len(s.block_table)]) == s.block_table
        assert (row[len(s.block_table):] == -1).all()
    assert len(np.unique(got["slot_mapping"])) == len(seqs)
    offsets, ids = ref.csr(seqs)
    c_got = c_oracle.pack_decode(
        [s.num_tokens for s in seqs], offsets, ids, bs, got["block_tables"].shape[1]
    )
    for key in ("slot_mapping", "context_lens", "block_tables", "cu_seqlens_k"):
        np.testing.assert_array_equal(c_got[key], got[key], err_msg=key)


def test_graph_replay_fill_keeps_stale_columns():
    buffers = {
        "slot_mapping": np.zeros(8, np.int32),
        "context_lens": np.full(8, 7, np.int32),
        "block_tables": np.full((8, 5), 9, np.int32),
    }
    ref.graph_replay_fill(buffers, np.array([3, 4], np.int32), np.array([10, 11], np.int32),
                          np.array([[1, 2], [3, -1]], np.int32))
    np.testing.assert_array_equal(buffers["slot_mapping"], [3, 4, -1, -1, -1, -1, -1, -1])
    np.testing.assert_array_equal(buffers["context_lens"], [10, 11, 0, 0, 0, 0, 0, 0])
    np.testing.assert_array_equal(buffers["block_tables"][:2], [[1, 2, 9, 9, 9], [3, -1, 9, 9, 9]])
    assert (buffers["block_tables"][2:] == 9).all()


# ------------------------------------------------------------ planted bugs

def test_goldens_catch_planted_store_mistakes():
    g = GOLDEN["store"]
    key, value = _arr(g["key"]), _arr(g["value"])
    slots = _arr(g["slot_mapping"], np.int32)

    def without_skip(k, v, kc, vc, s):  # treats -1 as the last row (python wrap-around)
        kc.reshape(-1, *kc.shape[2:])[s.astype(np.int64)] = k
        vc.reshape(-1, *vc.shape[2:])[s.astype(np.int64)] = v

    def swapped(k, v, kc, vc, s):  # K and V exchanged
        ref.store(v, k, kc, vc, s)

    for broken in (without_skip, swapped):
        kc = np.full(g["cache_shape"], -1, np.float32)
        vc = kc.copy()
        broken(key, value, kc, vc, slots)
        assert not (np.array_equal(kc, _arr(g["expected_key_cache"])) and
                    np.array_equal(vc, _arr(g["expected_value_cache"])))


def test_goldens_catch_planted_gather_mistakes():
    g = GOLDEN["gather"]
    cache = _arr(g["cache"])
    expected = _arr(g["expected"])
    bs = cache.shape[1]

    def off_by_one(c, table, length):  # ceil dropped: one block too few
        need = length // bs
        return c[np.asarray(table[:need])].reshape(-1, *c.shape[2:])[:length]

    def block_offset_swapped(c, table, length):  # out[t] = cache[table[t % BS], t // BS]
        return np.stack([c[table[t % bs], t // bs] for t in range(length)])

    for broken in (off_by_one, block_offset_swapped):
        try:
            got = broken(cache, g["block_table"], g["sequence_length"])
        except (IndexError, ValueError):
            continue
        assert got.shape != expected.shape or not np.array_equal(got, expected)
