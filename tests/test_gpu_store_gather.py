"""The fused prefill store + context gather (nkv_store_gather) against the
oracle's store followed by its varlen gather, bit-exact.

Covers the chunked-prefill and narrow-row workloads at full size (the
narrow-row step has requests whose cached prefix is in blocks another
request of the same step is filling), random prefill batches with shared
blocks, continuation chunks, empty requests and -1 slots, plans shared by
two layers, and a later step that must not see the previous step's
writers."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import c_oracle

pytestmark = pytest.mark.gpu

WORD = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}


def words(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(WORD[t.dtype]).numpy()


@pytest.fixture(scope="module")
def backend(gpu_device):
    from nanokv.paged_kv import create_paged_kv_backend

    return create_paged_kv_backend("hip")


def _compact(cache: torch.Tensor, blocks: np.ndarray):
    blocks = np.unique(blocks[blocks >= 0])
    index = torch.from_numpy(blocks.astype(np.int64)).to(cache.device)
    host = cache.index_select(0, index).cpu().contiguous().view(WORD[cache.dtype]).numpy()
    remap = np.full(cache.shape[0], -1, np.int64)
    remap[blocks] = np.arange(blocks.size)
    return host, remap


def _remap(tables: np.ndarray, slots: np.ndarray, remap: np.ndarray, bs: int):
    t = tables.astype(np.int64).copy()
    t[t >= 0] = remap[t[t >= 0]]
    s = slots.astype(np.int64).copy()
    s[s >= 0] = remap[s[s >= 0] // bs] * bs + s[s >= 0] % bs
    return t.astype(np.int32), s.astype(np.int32)


def _expect(hk, hv, key, value, tables, slots, cu_k):
    """The oracle's store, then its varlen gather of the stored caches."""
    c_oracle.store(key, value, hk, hv, slots, threads=8)
    return (c_oracle.gather_varlen(hk, tables, cu_k, threads=8),
            c_oracle.gather_varlen(hv, tables, cu_k, threads=8))


def _run_and_check(backend, device, kc, vc, key, value, tables, slots, cu_q, cu_k, *, plan=None):
    bs = kc.shape[1]
    used = np.concatenate([tables.ravel(), slots[slots >= 0] // bs])
    hk, remap = _compact(kc, used)
    hv, _ = _compact(vc, used)
    ctables, cslots = _remap(tables, slots, remap, bs)
    d = {name: torch.from_numpy(a).to(device) for name, a in
         (("tables", tables), ("slots", slots), ("cu_q", cu_q), ("cu_k", cu_k))}
    total = int(cu_k[-1])
    k_out, v_out = backend.store_gather(key, value, kc, vc, d["slots"], d["tables"], d["cu_q"],
                                        d["cu_k"], total, plan=plan)
    ek, ev = _expect(hk, hv, words(key), words(value), ctables, cslots, cu_k)
    np.testing.assert_array_equal(words(k_out), ek)
    np.testing.assert_array_equal(words(v_out), ev)
    got_k, _ = _compact(kc, used)
    got_v, _ = _compact(vc, used)
    np.testing.assert_array_equal(got_k, hk)
    np.testing.assert_array_equal(got_v, hv)


@pytest.mark.parametrize("name", ["chunked_prefill", "narrow_rows"])
def test_workload_full_size(backend, gpu_device, name):
    from nanokv import workloads

    wl = workloads.build(name)
    print(f"[store_gather {name}] seqs={wl.num_seqs} tokens={wl.slot_mapping.size}", flush=True)
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    g = torch.Generator(device=gpu_device).manual_seed(3)
    kc = torch.empty(shape, dtype=wl.dtype, device=gpu_device)
    kc.view(torch.int16).random_(-32768, 32767, generator=g)
    vc = torch.empty_like(kc)
    vc.view(torch.int16).random_(-32768, 32767, generator=g)
    cu_q = np.concatenate([[0], np.cumsum(wl.num_scheduled)]).astype(np.int32)
    _run_and_check(backend, gpu_device, kc, vc, wl.key.to(gpu_device), wl.value.to(gpu_device),
                   wl.padded_block_tables(), wl.slot_mapping, cu_q, wl.cu_seqlens_k())


def _prefill_batch(rng, num_seqs, bs, nb, *, share_in_step=True, minus_one=0, empty=True):
    """Requests with cached prefixes and new tokens, block lists from a
    permutation; with ``share_in_step`` odd requests take their first blocks
    from the previous request's blocks, which that request fills in this
    step (its cached prefix is then written in the same step)."""
    perm = list(rng.permutation(nb))
    tables, cached, scheduled = [], [], []
    for i in range(num_seqs):
        if share_in_step and i % 2 == 1 and scheduled[-1] > bs and cached[-1] == 0:
            share = int(rng.integers(1, scheduled[-1] // bs + 1))
            c = share * bs
            q = int(rng.integers(0 if empty else 1, 3 * bs))
            need = -(-(c + q) // bs)
            t = tables[-1][:share] + [perm.pop() for _ in range(need - share)]
        else:
            c = int(rng.integers(0, 3)) * bs + (int(rng.integers(0, bs)) if rng.random() < 0.3 else 0)
            q = int(rng.integers(0 if empty else 1, 4 * bs))
            need = -(-(c + q) // bs)
            t = [perm.pop() for _ in range(need)]
        tables.append(t)
        cached.append(c)
        scheduled.append(q)
    width = max(1, max(len(t) for t in tables))
    table = np.full((num_seqs, width + 1), -1, np.int32)
    for i, t in enumerate(tables):
        table[i, :len(t)] = t
    slots = []
    for t, c, q in zip(tables, cached, scheduled):
        for p in range(c, c + q):
            slots.append(t[p // bs] * bs + p % bs)
    slots = np.asarray(slots, np.int32)
    if minus_one and slots.size:
        slots[rng.choice(slots.size, min(minus_one, slots.size), replace=False)] = -1
    cu_q = np.concatenate([[0], np.cumsum(scheduled)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(np.asarray(cached) + np.asarray(scheduled))]).astype(np.int32)
    return table, slots, cu_q, cu_k


@pytest.mark.parametrize("dtype,heads,dim,bs,seed", [
    (torch.bfloat16, 8, 128, 256, 1),
    (torch.bfloat16, 2, 128, 256, 2),
    (torch.float16, 2, 128, 16, 3),
    (torch.float32, 1, 64, 16, 4),
    (torch.float16, 3, 5, 4, 5),
])
@pytest.mark.parametrize("minus_one", [0, 9])
def test_random_prefill_batches(backend, gpu_device, dtype, heads, dim, bs, seed, minus_one):
    rng = np.random.default_rng(seed * 100 + minus_one)
    nb = 4000
    table, slots, cu_q, cu_k = _prefill_batch(rng, 23, bs, nb, minus_one=minus_one)
    g = torch.Generator(device=gpu_device).manual_seed(seed)
    kc = torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(dtype)
    vc = torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(dtype)
    t = int(cu_q[-1])
    key = torch.randn(t, heads, dim, device=gpu_device, generator=g).to(dtype)
    value = torch.randn(t, heads, dim, device=gpu_device, generator=g).to(dtype)
    print(f"[store_gather random] {dtype} {heads}x{dim} bs={bs} tokens={t} rows={int(cu_k[-1])}",
          flush=True)
    _run_and_check(backend, gpu_device, kc, vc, key, value, table, slots, cu_q, cu_k)


def test_fused_qkv_views_and_one_plan_for_two_layers(backend, gpu_device):
    """K/V as strided views of a fused QKV output; the plan built once
    serves two layers' caches."""
    rng = np.random.default_rng(77)
    bs, heads, dim, nb = 16, 2, 128, 600
    table, slots, cu_q, cu_k = _prefill_batch(rng, 9, bs, nb)
    t = int(cu_q[-1])
    g = torch.Generator(device=gpu_device).manual_seed(9)
    qkv = torch.randn(t, (8 + 2 * heads) * dim, device=gpu_device, generator=g).to(torch.bfloat16)
    _, k, v = qkv.split([8 * dim, heads * dim, heads * dim], dim=-1)
    key, value = k.view(t, heads, dim), v.view(t, heads, dim)
    assert key.stride(0) != heads * dim
    caches = [torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(torch.bfloat16)
              for _ in range(4)]
    d_tables = torch.from_numpy(table).to(gpu_device)
    plan = backend.build_store_gather_plan(caches[0], d_tables, torch.from_numpy(cu_q).to(gpu_device),
                                           torch.from_numpy(cu_k).to(gpu_device), t, int(cu_k[-1]))
    for layer in range(2):
        _run_and_check(backend, gpu_device, caches[2 * layer], caches[2 * layer + 1], key, value,
                       table, slots, cu_q, cu_k, plan=plan)


def test_next_step_ignores_previous_writers(backend, gpu_device):
    """Step A writes blocks that its other requests read as cached prefix;
    step B reads those blocks as plain cached rows (nobody writes them in
    B), so B must take them from the cache, not from A's tokens."""
    rng = np.random.default_rng(5)
    bs, heads, dim, nb = 16, 2, 64, 800
    g = torch.Generator(device=gpu_device).manual_seed(5)
    kc = torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(torch.float16)
    vc = torch.randn_like(kc)
    table, slots, cu_q, cu_k = _prefill_batch(rng, 12, bs, nb)
    t = int(cu_q[-1])
    key = torch.randn(t, heads, dim, device=gpu_device, generator=g).to(torch.float16)
    value = torch.randn_like(key)
    _run_and_check(backend, gpu_device, kc, vc, key, value, table, slots, cu_q, cu_k)
    # step B: the same requests continue with one new token each (their
    # previous rows are now all cached)
    lens = np.diff(cu_k)
    new_tables, new_slots = table.copy(), []
    spare = iter(range(nb - 1, -1, -1))
    used = set(table[table >= 0].tolist())
    for i, n in enumerate(lens.tolist()):
        if n % bs == 0:
            block = next(b for b in spare if b not in used)
            used.add(block)
            col = int((new_tables[i] >= 0).sum())
            if col >= new_tables.shape[1]:
                new_tables = np.concatenate([new_tables, np.full((len(lens), 1), -1, np.int32)], 1)
            new_tables[i, col] = block
        new_slots.append(int(new_tables[i, n // bs]) * bs + n % bs)
    cu_q_b = np.arange(len(lens) + 1, dtype=np.int32)
    cu_k_b = np.concatenate([[0], np.cumsum(lens + 1)]).astype(np.int32)
    key_b = torch.randn(len(lens), heads, dim, device=gpu_device, generator=g).to(torch.float16)
    value_b = torch.randn_like(key_b)
    _run_and_check(backend, gpu_device, kc, vc, key_b, value_b, new_tables,
                   np.asarray(new_slots, np.int32), cu_q_b, cu_k_b)


def test_empty_step_and_context_only(backend, gpu_device):
    """No new tokens at all (a gather of cached contexts), and no rows."""
    bs, nb = 16, 64
    kc = torch.randn(nb, bs, 2, 64, device=gpu_device).to(torch.bfloat16)
    vc = torch.randn_like(kc)
    table = np.array([[3, 7, -1], [5, -1, -1]], np.int32)
    cu_q = np.zeros(3, np.int32)
    cu_k = np.array([0, 20, 31], np.int32)
    empty = torch.empty(0, 2, 64, device=gpu_device, dtype=torch.bfloat16)
    _run_and_check(backend, gpu_device, kc, vc, empty, empty.clone(), table,
                   np.zeros(0, np.int32), cu_q, cu_k)
    k_out, v_out = backend.store_gather(
        empty, empty.clone(), kc, vc, torch.zeros(0, dtype=torch.int32, device=gpu_device),
        torch.from_numpy(table).to(gpu_device), torch.zeros(3, dtype=torch.int32, device=gpu_device),
        torch.zeros(3, dtype=torch.int32, device=gpu_device), 0)
    assert k_out.shape == (0, 2, 64) and v_out.shape == (0, 2, 64)


def _expected_plan(tables, cu_q, cu_k, bs, chunk, num_blocks):
    """The plan restated on the host: per token {output row, slot of its
    position}; per cached chunk {source row, output row, rows, request} and
    {token of the chunk's first row, [lo, hi) rows written in this step}."""
    num_seqs = len(cu_q) - 1
    meta, writer = [], {}
    for t in range(int(cu_q[-1])):
        i = int(np.searchsorted(cu_q, t, side="right")) - 1
        lk, lq = int(cu_k[i + 1] - cu_k[i]), int(cu_q[i + 1] - cu_q[i])
        p = lk - lq + t - int(cu_q[i])
        block = int(tables[i, p // bs]) if p // bs < tables.shape[1] else -1
        slot = block * bs + p % bs if 0 <= block < num_blocks else -1
        meta.append((int(cu_k[i]) + p, slot))
        if slot >= 0 and (p % bs == 0 or t == cu_q[i]):
            writer[block] = (i, p // bs)
    entries = []
    for i in range(num_seqs):
        cached = int(cu_k[i + 1] - cu_k[i]) - int(cu_q[i + 1] - cu_q[i])
        for row0 in range(0, max(cached, 0), chunk):
            rows = min(chunk, cached - row0)
            block = int(tables[i, row0 // bs]) if row0 // bs < tables.shape[1] else -1
            src = block * bs + row0 % bs if 0 <= block < num_blocks else -1
            tail = (0, 0, 0, 0)
            if src >= 0 and block in writer:
                w, wl = writer[block]
                wlk = int(cu_k[w + 1] - cu_k[w])
                wstart = wlk - int(cu_q[w + 1] - cu_q[w])
                first = wl * bs + row0 % bs
                lo = max(0, min(rows, wstart - first))
                hi = max(lo, min(rows, wlk - first))
                if lo < hi:
                    tail = (int(cu_q[w]) + first - wstart, lo, hi, 0)
            entries.append((src, int(cu_k[i]) + row0, rows, i) + tail)
    return meta, entries


@pytest.mark.parametrize("source", ["narrow_rows", "random"])
def test_plan_marks_rows_written_in_the_step(backend, gpu_device, source):
    """The plan, read back, equals its host restatement: every cached chunk
    whose rows another request writes in this step names that token range
    (the fused launch takes those rows from K/V, never from the cache)."""
    from nanokv import _lib, workloads

    if source == "narrow_rows":
        wl = workloads.build("narrow_rows")
        tables, cu_q, cu_k = wl.padded_block_tables(), wl.cu_seqlens_q(), wl.cu_seqlens_k()
        bs, nb, heads, dim = wl.block_size, wl.num_blocks, wl.num_kv_heads, wl.head_dim
    else:
        rng = np.random.default_rng(31)
        bs, nb, heads, dim = 16, 3000, 2, 128
        tables, _, cu_q, cu_k = _prefill_batch(rng, 31, bs, nb)
    cache = torch.empty((nb, bs, heads, dim), dtype=torch.bfloat16, device=gpu_device)
    t, total = int(cu_q[-1]), int(cu_k[-1])
    plan = backend.build_store_gather_plan(
        cache, torch.from_numpy(tables).to(gpu_device), torch.from_numpy(cu_q).to(gpu_device),
        torch.from_numpy(cu_k).to(gpu_device), t, total).cpu().numpy()
    chunk = _lib.load_library().nkv_gather_plan_rows(bs, heads * dim, _lib.NKV_DTYPE_BFLOAT16)
    meta, entries = _expected_plan(tables, cu_q, cu_k, bs, chunk, nb)
    meta_words = (t * 8 + 15) // 16 * 4
    np.testing.assert_array_equal(plan[:2 * t].reshape(t, 2), np.asarray(meta, np.int32).reshape(t, 2))
    got = plan[meta_words:].reshape(-1, 8)
    assert len(entries) <= got.shape[0]
    np.testing.assert_array_equal(got[:len(entries)], np.asarray(entries, np.int32).reshape(-1, 8))
    assert (got[len(entries):] == 0).all()
    written = sum(1 for e in entries if e[6] > e[5])
    print(f"[store_gather plan {source}] {len(entries)} cached chunks, {written} with rows written "
          f"in the step", flush=True)
    assert written > 0


def test_decode_step_shape(backend, gpu_device):
    """One new token per sequence (the decode step through the fused op):
    256 contexts log-uniform in [256, 16384] at full size, then a small
    batch whose last rows are graph-bucket padding as the decode graph's
    replay fill leaves them (model_runner.py:993-1011): a token with slot -1
    and context length 0, so it is neither stored nor gathered."""
    from nanokv import workloads

    wl = workloads.build("decode_step", num_layers=1)
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    g = torch.Generator(device=gpu_device).manual_seed(8)
    kc = torch.empty(shape, dtype=wl.dtype, device=gpu_device)
    kc.view(torch.int16).random_(-32768, 32767, generator=g)
    vc = torch.empty_like(kc)
    vc.view(torch.int16).random_(-32768, 32767, generator=g)
    cu_q = np.arange(wl.num_seqs + 1, dtype=np.int32)
    print(f"[store_gather decode] seqs={wl.num_seqs} rows={int(wl.num_tokens.sum())}", flush=True)
    _run_and_check(backend, gpu_device, kc, vc, wl.key[0].to(gpu_device), wl.value[0].to(gpu_device),
                   wl.padded_block_tables(), wl.slot_mapping, cu_q, wl.cu_seqlens_k())

    bs, nb = 16, 64
    kc = torch.randn(nb, bs, 2, 64, device=gpu_device, generator=g).to(torch.float16)
    vc = torch.randn_like(kc)
    table = np.array([[5, 9, -1], [11, -1, -1], [-1, -1, -1], [-1, -1, -1]], np.int32)
    lens = np.array([20, 3, 0, 0])                      # the last two are padding rows
    slots = np.array([9 * bs + 3, 11 * bs + 2, -1, -1], np.int32)
    cu_q = np.arange(5, dtype=np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    key = torch.randn(4, 2, 64, device=gpu_device, generator=g).to(torch.float16)
    value = torch.randn_like(key)
    _run_and_check(backend, gpu_device, kc, vc, key, value, table, slots, cu_q, cu_k)
