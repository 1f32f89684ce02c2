"""The fused prefill store + context gather (nkv_store_gather) against the
oracle's store followed by its varlen gather, bit-exact.

Covers the chunked-prefill and narrow-row workloads at full size (the
narrow-row step in the reference's order: duplicated-image requests hit
prefix blocks filled and hashed in an earlier step), random prefill batches
whose requests share earlier-step prefix blocks, continuation chunks, empty
requests and -1 slots, plans shared by two layers, two consecutive steps,
the decode shape, the plan's layout, and plans or inputs the op must
reject before any launch."""
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


def _prefill_batch(rng, num_seqs, bs, nb, *, share=True, minus_one=0, empty=True):
    """Requests with cached prefixes and new tokens, block lists from a
    permutation.  With ``share``, an odd request whose predecessor holds full
    cached blocks reuses some of them as its own cached prefix: blocks the
    predecessor filled in an earlier step, hashed after that step, as the
    reference's prefix cache hands them out (scheduler.py:196-200,
    block_manager.py:119-198,229-258), so no new row of the batch lands in
    any request's cached prefix."""
    perm = list(rng.permutation(nb))
    tables, cached, scheduled = [], [], []
    for i in range(num_seqs):
        if share and i % 2 == 1 and cached[-1] >= bs:
            hit = int(rng.integers(1, cached[-1] // bs + 1))
            c = hit * bs
            q = int(rng.integers(0 if empty else 1, 3 * bs))
            need = max(hit, -(-(c + q) // bs))
            t = tables[-1][:hit] + [perm.pop() for _ in range(need - hit)]
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


def _cached_rows_untouched(table, slots, cu_q, cu_k, bs) -> bool:
    """No request's cached prefix holds a slot that the batch stores."""
    written = set(slots[slots >= 0].tolist())
    for i in range(len(cu_q) - 1):
        cached = int(cu_k[i + 1] - cu_k[i]) - int(cu_q[i + 1] - cu_q[i])
        for p in range(cached):
            if int(table[i, p // bs]) * bs + p % bs in written:
                return False
    return True


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
    assert _cached_rows_untouched(table, slots, cu_q, cu_k, bs)
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


def test_two_consecutive_steps(backend, gpu_device):
    """Step A stores its requests' new rows; in step B the same requests
    continue with one new token each, and every row A stored is now part of
    a cached prefix that B's launch copies from the cache."""
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
    position}; per cached chunk {source row, output row, rows, request}."""
    num_seqs = len(cu_q) - 1
    meta = []
    for t in range(int(cu_q[-1])):
        i = int(np.searchsorted(cu_q, t, side="right")) - 1
        lk, lq = int(cu_k[i + 1] - cu_k[i]), int(cu_q[i + 1] - cu_q[i])
        p = lk - lq + t - int(cu_q[i])
        block = int(tables[i, p // bs]) if p // bs < tables.shape[1] else -1
        slot = block * bs + p % bs if 0 <= block < num_blocks else -1
        meta.append((int(cu_k[i]) + p, slot))
    entries = []
    for i in range(num_seqs):
        cached = int(cu_k[i + 1] - cu_k[i]) - int(cu_q[i + 1] - cu_q[i])
        for row0 in range(0, max(cached, 0), chunk):
            rows = min(chunk, cached - row0)
            block = int(tables[i, row0 // bs]) if row0 // bs < tables.shape[1] else -1
            src = block * bs + row0 % bs if 0 <= block < num_blocks else -1
            entries.append((src, int(cu_k[i]) + row0, rows, i))
    return meta, entries


@pytest.mark.parametrize("source", ["narrow_rows", "random"])
def test_plan_matches_host_restatement(backend, gpu_device, source):
    """The plan, read back, equals its host restatement: every token's
    output row and slot, every cached-prefix chunk, zeros past the last."""
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
    got = plan[meta_words:].reshape(-1, 4)
    assert 0 < len(entries) <= got.shape[0]
    np.testing.assert_array_equal(got[:len(entries)], np.asarray(entries, np.int32).reshape(-1, 4))
    assert (got[len(entries):] == 0).all()
    print(f"[store_gather plan {source}] {t} tokens, {len(entries)} cached chunks", flush=True)


def test_plan_and_inputs_rejected_before_launch(backend, gpu_device):
    """A plan built for other token or context counts, an int64 or short
    slot_mapping, and a key narrower than the cache's rows all raise on the
    host; the caches and outputs stay as they were."""
    from nanokv.paged_kv import ops

    rng = np.random.default_rng(12)
    bs, heads, dim, nb = 16, 2, 64, 300
    table, slots, cu_q, cu_k = _prefill_batch(rng, 6, bs, nb, empty=False)
    t, total = int(cu_q[-1]), int(cu_k[-1])
    g = torch.Generator(device=gpu_device).manual_seed(12)
    kc = torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(torch.bfloat16)
    vc = torch.randn_like(kc)
    before_k, before_v = kc.clone(), vc.clone()
    key = torch.randn(t, heads, dim, device=gpu_device, generator=g).to(torch.bfloat16)
    value = torch.randn_like(key)
    d_tables = torch.from_numpy(table).to(gpu_device)
    d_cu_q, d_cu_k = torch.from_numpy(cu_q).to(gpu_device), torch.from_numpy(cu_k).to(gpu_device)
    d_slots = torch.from_numpy(slots).to(gpu_device)
    k_out = torch.zeros(total, heads, dim, device=gpu_device, dtype=torch.bfloat16)
    v_out = torch.zeros_like(k_out)
    n = len(cu_q) - 1
    good = backend.build_store_gather_plan(kc, d_tables, d_cu_q, d_cu_k, t, total)
    # (8 bytes of plan per token, in 16-byte steps: two more tokens move the chunk entries)
    wrong = [backend.build_store_gather_plan(kc, d_tables, d_cu_q, d_cu_k, t + 2, total),
             backend.build_store_gather_plan(kc, d_tables, d_cu_q, d_cu_k, t, total + 4 * 1024)]
    for plan in wrong:
        with pytest.raises(ValueError, match="plan"):
            backend.store_gather(key, value, kc, vc, d_slots, d_tables, d_cu_q, d_cu_k, total,
                                 plan=plan, out=(k_out, v_out))
        with pytest.raises(ValueError, match="plan"):
            ops.store_gather(key, value, kc, vc, d_slots, plan, n, k_out, v_out)
    bad_inputs = [
        (key, value, d_slots.long(), "int32"),                   # int64 slots
        (key, value, d_slots[:-1], "one slot per token"),        # short slot_mapping
        (key[:, :1], value[:, :1], d_slots, "must match"),       # fewer kv heads than the cache
    ]
    for k, v, sl, message in bad_inputs:
        with pytest.raises(RuntimeError, match=message):
            ops.store_gather(k, v, kc, vc, sl, good, n, k_out, v_out)
        with pytest.raises(RuntimeError, match=message):
            torch.ops.nanovllm_paged_kv.store_gather(k, v, kc, vc, sl, good, n, k_out, v_out)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), before_k.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), before_v.view(torch.int16))
    assert not k_out.view(torch.int16).any() and not v_out.view(torch.int16).any()
    # the good plan still runs, and the op matches the oracle
    _run_and_check(backend, gpu_device, kc, vc, key, value, table, slots, cu_q, cu_k, plan=good)


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
