"""Paged-attention decode on the GPU vs the float32 oracle
(oracle.paged_kv.paged_attention_decode, itself pinned to torch's SDPA with
GQA in tests/test_attention_oracle.py).

Two MFMA kernels serve the layouts (1-16 query heads per kv head): below 8
kv heads the range split (the contexts in 16-row chunks laid end to end,
cut into equal ranges for 1024 / Hkv worker wavefronts per kv head, ranges
crossing sequence boundaries), from 8 kv heads on the entry split (one
workgroup per 768-row entry of one sequence and kv head).  Scores and the
softmax run in fp32; the kernels round the weights p to bf16 / fp16 before
the second product (as flash attention does) and round the result once.
Each rounding is <= 2^-9 relative, so an element differs from the fp32 result by
at most 2^-9 * sum_k p_k |v_k| / sum_k p_k (the same attention over |V|,
"ref_abs") plus 2^-9 * |ref|; the tests allow 1e-3 + 2^-8 * (ref_abs + |ref|)
(the fp16 partial sums of the split-K merge keep 12 bits relative to each
head's largest value, well inside the 1e-3).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as oracle

pytestmark = pytest.mark.gpu

ATOL = 1e-3


@pytest.fixture(scope="module")
def backend(gpu_device):
    from nanokv.paged_kv import create_paged_kv_backend

    return create_paged_kv_backend("hip")


def reference(host, scale, dtype="bfloat16"):
    """The oracle's output and the same attention over |V| (sign bits cleared)."""
    args = (host["q"], host["kc"])
    tail = (host["tables"], host["lens"], scale)
    ref = oracle.paged_attention_decode(*args, host["vc"], *tail, dtype=dtype)
    ref_abs = oracle.paged_attention_decode(*args, host["vc"] & np.int16(0x7FFF), *tail, dtype=dtype)
    return ref, ref_abs


def check_close(got: torch.Tensor, expected, what: str) -> None:
    ref, ref_abs = expected
    g = got.float().cpu().numpy()
    bad = np.abs(g - ref) > ATOL + 2.0 ** -8 * (ref_abs + np.abs(ref))
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {np.abs(g - ref).max():.3e}"


def build_case(device, hkv, g, bs, lens, seed, q_pad_heads=0, dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    b = len(lens)
    need = [-(-int(n) // bs) for n in lens]
    nb = sum(need) + 5
    width = max(1, max(need))
    perm = torch.randperm(nb, generator=gen).numpy()
    tables = np.full((b, width), -1, np.int32)
    cursor = 0
    for i, n in enumerate(need):
        tables[i, :n] = perm[cursor:cursor + n]
        cursor += n
    kc = torch.randn(nb, bs, hkv, 128, generator=gen).to(dtype)
    vc = torch.randn(nb, bs, hkv, 128, generator=gen).to(dtype)
    hq = hkv * g
    q_full = torch.randn(b, hq + q_pad_heads, 128, generator=gen).to(dtype)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    dev = dict(
        kc=kc.to(device), vc=vc.to(device), q=q_full.to(device)[:, :hq],
        tables=torch.from_numpy(tables).to(device), cu=torch.from_numpy(cu).to(device),
    )
    host = dict(q=q_full[:, :hq].float().numpy(), kc=kc.view(torch.int16).numpy(),
                vc=vc.view(torch.int16).numpy(), tables=tables, lens=np.asarray(lens))
    return dev, host, int(cu[-1])


@pytest.mark.parametrize("hkv,g,bs", [
    (8, 2, 256), (8, 2, 16), (2, 8, 256), (2, 8, 16), (4, 4, 16), (4, 2, 32),
    (8, 1, 16), (2, 1, 16), (1, 8, 16), (1, 1, 4), (2, 4, 8),
    (8, 2, 24), (2, 4, 1000),  # block sizes that are not powers of two (1000: entries of 500 rows)
    (8, 4, 16), (4, 7, 256), (4, 8, 16), (8, 3, 16), (2, 5, 8), (1, 6, 16),  # up to 32 query heads
    (8, 5, 16), (8, 8, 256),  # 40 and 64 query heads
    (2, 16, 16), (1, 12, 256), (4, 10, 24), (2, 9, 8),  # 9-16 query heads per kv head
    (3, 4, 16), (16, 2, 16), (6, 1, 32), (5, 3, 256),  # kv-head counts other than 1, 2, 4, 8
])
def test_decode_attention_matches_oracle(backend, gpu_device, hkv, g, bs):
    lens = [0, 1, bs - 1, bs, bs + 1, 3 * bs + 7, 2, 5 * bs, 17, 1]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv * 100 + g * 10 + bs)
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, scale)
    ref = reference(host, scale)
    check_close(out, ref, f"hkv={hkv} g={g} bs={bs}")
    assert torch.all(out[0] == 0), "an empty context must give zeros"


@pytest.mark.parametrize("hkv,g,bs", [
    (8, 2, 16), (2, 8, 256), (1, 1, 4), (4, 2, 24), (8, 6, 16), (2, 16, 16), (3, 4, 24)])
def test_decode_attention_float16_matches_oracle(backend, gpu_device, hkv, g,
                                                 bs):
    """float16 q and caches (the fp16 MFMAs), fp16 output; the same
    tolerance holds (fp16 rounds to 2^-11)."""
    lens = [0, 1, bs - 1, bs, bs + 1, 3 * bs + 7, 2, 5 * bs, 17, 1]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv + g + bs,
                                  dtype=torch.float16)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, 0.0884)
    assert out.dtype == torch.float16
    ref = reference(host, 0.0884, "float16")
    check_close(out, ref, f"fp16 hkv={hkv} g={g} bs={bs}")


@pytest.mark.parametrize("hkv,g", [(8, 2), (2, 8)])
def test_strided_q_plan_reuse_and_out_buffer(backend, gpu_device, hkv, g):
    """q with padding heads (row stride past Hq * 128), one plan reused by
    two calls, and a caller-owned output buffer."""
    lens = [300, 1, 513, 256, 40]
    dev, host, total = build_case(gpu_device, hkv, g, 256, lens, seed=7, q_pad_heads=16)
    assert dev["q"].stride(0) == (hkv * g + 16) * 128
    plan = backend.build_attention_plan(dev["kc"], dev["cu"], total)
    out = torch.empty((len(lens), hkv * g, 128), dtype=torch.bfloat16, device=gpu_device)
    ref = reference(host, 0.1)
    for _ in range(2):
        out.zero_()
        backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                       total, 0.1, plan=plan, out=out)
        check_close(out, ref, "planned")


def test_unsupported_decode_layouts_raise(backend, gpu_device):
    """More than 16 query heads per kv head raises."""
    lens = [5, 9]
    for hkv, g in ((8, 17), (1, 32)):
        dev, _, total = build_case(gpu_device, hkv, 1, 16, lens, seed=4)
        q = torch.zeros((2, hkv * g, 128), dtype=torch.bfloat16, device=gpu_device)
        with pytest.raises((ValueError, RuntimeError), match="head layout"):
            backend.paged_attention_decode(q, dev["kc"], dev["vc"], dev["tables"], dev["cu"], total,
                                           0.1)


def test_plan_for_other_lengths_is_rejected(backend, gpu_device):
    """A plan sized for shorter contexts cannot cover these: refused on the
    host instead of leaving rows out."""
    lens = [300, 1, 513, 256, 40]
    dev, _, total = build_case(gpu_device, 8, 2, 16, lens, seed=9)
    short = torch.tensor([0, 1, 2, 3, 4, 5], dtype=torch.int32, device=gpu_device)
    plan = backend.build_attention_plan(dev["kc"], short, 5)
    with pytest.raises(ValueError, match="attention plan"):
        backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                       total, 0.1, plan=plan)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_range_plan_for_other_kv_heads_gives_nan(backend, gpu_device, dtype):
    """A range plan built for 2 kv heads, passed straight to the registered
    op with a 4-kv-head cache (the host check of AttentionPlan bypassed):
    the range kernel writes no partial, and the merge turns every output
    into NaN instead of returning stale workspace values."""
    lens = [300, 1, 513, 256, 40]
    two, _, total = build_case(gpu_device, 2, 4, 16, lens, seed=12, dtype=dtype)
    four, _, _ = build_case(gpu_device, 4, 2, 16, lens, seed=13, dtype=dtype)
    plan = backend.build_attention_plan(two["kc"], two["cu"], total)
    out = torch.zeros_like(four["q"])
    torch.ops.nanovllm_paged_kv.paged_attention_decode(
        four["q"], four["kc"], four["vc"], four["tables"], plan[0], plan[1], 0.1, out)
    assert torch.isnan(out.float()).all()
    with pytest.raises(ValueError, match="attention plan was built for"):
        backend.paged_attention_decode(four["q"], four["kc"], four["vc"], four["tables"], four["cu"],
                                       total, 0.1, plan=plan)


WORKERS = 1024  # worker wavefronts per launch of the range split: 1024 / Hkv per kv head
ENTRY_MIN_KV_HEADS = 8  # kv heads from which the entry split runs
SEG_COST = 1  # units the split charges for starting a sequence
KEYS = 16  # context rows per chunk


def expected_attention_plan(lens, hkv):
    """The decode plan restated.  Each non-empty sequence takes SEG_COST
    start-up units, then one unit per 16-row chunk, laid end to end over all
    sequences; the U units are cut into W = min(WORKERS // hkv, U) equal ranges
    [w U / W, (w + 1) U / W).  Record w = {sequence of its first unit, its
    first chunk there, its end unit, 0}; vstart[i] = unit of sequence i's
    chunk 0; a sequence's partials are numbered by worker, from first[i]."""
    n = len(lens)
    chunks = np.array([-(-int(x) // KEYS) for x in lens], np.int64)
    units = np.where(chunks > 0, chunks + SEG_COST, 0)
    ustart = np.concatenate([[0], np.cumsum(units)]).astype(np.int64)
    total = int(ustart[-1])
    workers = min(max(1, WORKERS // hkv), total)

    def worker_of(v):
        return ((v + 1) * workers - 1) // total

    parts = [0 if c == 0 else worker_of(ustart[i + 1] - 1) - worker_of(ustart[i] + SEG_COST) + 1
             for i, c in enumerate(chunks)]
    first = np.concatenate([[0], np.cumsum(parts)]).astype(np.int64)
    records = np.zeros((WORKERS, 4), np.int64)
    for w in range(workers):
        b, e = w * total // workers, (w + 1) * total // workers
        s = int(np.searchsorted(ustart[:n], b, side="right")) - 1
        records[w] = (s, max(0, b - ustart[s] - SEG_COST), e, 0)
    return dict(header=(workers, total, n, hkv), records=records, lens=np.asarray(lens, np.int64),
                vstart=ustart[:n] + SEG_COST, first=first)


def expected_entry_plan(lens, rows):
    """The entry split's plan restated: sequence by sequence, entries of
    `rows` context rows in row order (the last one short when rows does not
    divide the length), {row0, rows, seq, 0}; first entry of each
    sequence."""
    first = np.concatenate([[0], np.cumsum([-(-n // rows) for n in lens])]).astype(np.int64)
    entries = [(r, min(rows, n - r), i, 0) for i, n in enumerate(lens) for r in range(0, n, rows)]
    return np.array(entries, dtype=np.int64).reshape(-1, 4), first


def check_entry_plan(plan, first, lens, rows):
    expect, expect_first = expected_entry_plan(lens, rows)
    got = plan.cpu().numpy().astype(np.int64)
    np.testing.assert_array_equal(first.cpu().numpy(), expect_first)
    np.testing.assert_array_equal(got[: len(expect)], expect)
    assert not got[len(expect):, 1].any()  # entries past the total are empty


def read_attention_plan(plan, first, num_seqs):
    """The plan tensor's parts: header, worker records, lens, vstart."""
    flat = plan.cpu().numpy().astype(np.int64).reshape(-1)
    words = 4 * (-(-num_seqs // 4))
    base = 4 * (1 + WORKERS)
    return dict(header=tuple(flat[:4]), records=flat[4:base].reshape(WORKERS, 4),
                lens=flat[base:base + num_seqs], vstart=flat[base + words:base + words + num_seqs],
                first=first.cpu().numpy().astype(np.int64))


def walk_attention_plan(p):
    """The chunks each worker computes and the partials it writes, walked as
    the kernel's worker walks its range: from (seq, chunk0) on, up to the
    end unit, into the next non-empty sequence when one runs out.  Asserts
    that every chunk of every context is computed exactly once, that each
    sequence's partials are exactly first[i] .. first[i + 1] - 1, and that
    no worker holds more than its share of units.  Returns the chunk count
    per worker."""
    workers, total, n, _ = p["header"]
    lens, vstart, first = p["lens"], p["vstart"], p["first"]
    seen = np.zeros(int(sum(-(-int(x) // KEYS) for x in lens)), np.int64)
    offset = np.concatenate([[0], np.cumsum([-(-int(x) // KEYS) for x in lens])])
    owner = {}
    per_worker = []
    for w in range(workers):
        s, c, end, _ = (int(x) for x in p["records"][w])
        count = 0
        if lens[s] > 0 and vstart[s] + c < end:
            part = int(first[s]) + w - ((int(vstart[s]) + 1) * workers - 1) // total
            while True:
                nch = -(-int(lens[s]) // KEYS)
                while c < nch and vstart[s] + c < end:
                    seen[offset[s] + c] += 1
                    c += 1
                    count += 1
                assert part not in owner, f"partial {part} written twice"
                owner[part] = s
                if c < nch:
                    break
                s2 = s + 1
                while s2 < n and lens[s2] == 0:
                    s2 += 1
                if s2 >= n or vstart[s2] >= end:
                    break
                s, c, part = s2, 0, int(first[s2])
        per_worker.append(count)
    assert (seen == 1).all(), "a chunk is computed twice or never"
    for i in range(n):
        assert sorted(p for p, s in owner.items() if s == i) == list(range(first[i], first[i + 1]))
    assert max(per_worker, default=0) <= -(-total // max(workers, 1))
    return per_worker


@pytest.mark.parametrize("hkv,g,bs", [
    (8, 2, 16), (2, 4, 8), (4, 2, 4), (1, 1, 1024), (8, 4, 4), (2, 8, 1024)])
def test_long_contexts_over_small_blocks(backend, gpu_device, hkv, g, bs):
    """Contexts of hundreds to thousands of rows over blocks of 4-16 rows
    (a range or an entry spans tens of blocks) or inside one 1024-row block,
    with ragged tails.  Range split (below 8 kv heads): the plan equals its
    restatement and its walk covers every chunk once.  Entry split (8 kv
    heads): entries of nkv_attention_entry_rows rows tile each context in
    order."""
    from nanokv import _lib

    lens = [2309, 768, 769, 1535, 7, 1]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv * 7 + g + bs)
    plan, first = backend.build_attention_plan(dev["kc"], dev["cu"], total)
    if hkv >= ENTRY_MIN_KV_HEADS:
        check_entry_plan(plan, first, lens, int(_lib.load_library().nkv_attention_entry_rows(bs)))
    else:
        got = read_attention_plan(plan, first, len(lens))
        expect = expected_attention_plan(lens, hkv)
        for key in ("header", "records", "lens", "vstart", "first"):
            np.testing.assert_array_equal(np.asarray(got[key]), np.asarray(expect[key]), err_msg=key)
        walk_attention_plan(got)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, 1 / math.sqrt(128), plan=(plan, first))
    ref = reference(host, 1 / math.sqrt(128))
    check_close(out, ref, f"hkv={hkv} g={g} bs={bs}")


@pytest.mark.parametrize("hkv,g", [(8, 2), (2, 8), (1, 1), (4, 16)])
@pytest.mark.parametrize("lens", [[0], [0, 0, 0], [1], [1, 1, 1], [0, 1, 0], [16], [17, 0]])
def test_empty_and_tiny_batches(backend, gpu_device, hkv, g, lens):
    """Every context empty (the range split has no units and no workers;
    each output row must be zeros), and one-token or one-chunk contexts
    (worker ranges of a start-up unit and at most two chunks)."""
    dev, host, total = build_case(gpu_device, hkv, g, 16, lens, seed=31 + sum(lens))
    out = torch.full_like(dev["q"], float("nan"))
    backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                   total, 0.1, out=out)
    check_close(out, reference(host, 0.1), f"hkv={hkv} g={g} lens={lens}")
    for i, n in enumerate(lens):
        if n == 0:
            assert torch.all(out[i] == 0), f"empty context {i} must give zeros"


@pytest.mark.parametrize("hkv,g", [(8, 2), (2, 8)])
def test_no_sequences(backend, gpu_device, hkv, g):
    """A batch of no sequences: an empty output, no launch reads a plan."""
    kc = torch.zeros((4, 16, hkv, 128), dtype=torch.bfloat16, device=gpu_device)
    tables = torch.zeros((0, 1), dtype=torch.int32, device=gpu_device)
    cu = torch.zeros(1, dtype=torch.int32, device=gpu_device)
    q = torch.zeros((0, hkv * g, 128), dtype=torch.bfloat16, device=gpu_device)
    out = backend.paged_attention_decode(q, kc, kc, tables, cu, 0, 0.1)
    assert out.shape == (0, hkv * g, 128)


def test_plan_at_the_sequence_limit(backend, gpu_device):
    """NKV_MAX_PLAN_SEQS (8192) sequences, lengths 0 .. 3000: the plan
    kernel's LDS scan at its largest; the whole plan equals the
    restatement, workers past the split are empty, and the walk covers
    every chunk once with each worker within its share."""
    rng = np.random.default_rng(81)
    lens = rng.integers(0, 3001, 8192)
    lens[:7] = [0, 768, 769, 767, 1, 1536, 0]
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)).to(gpu_device)
    cache = torch.empty((1, 16, 1, 128), dtype=torch.bfloat16, device=gpu_device)
    plan, first = backend.build_attention_plan(cache, cu, int(lens.sum()))
    got = read_attention_plan(plan, first, len(lens))
    expect = expected_attention_plan(lens.tolist(), 1)
    for key in ("header", "records", "lens", "vstart", "first"):
        np.testing.assert_array_equal(np.asarray(got[key]), np.asarray(expect[key]), err_msg=key)
    per_worker = walk_attention_plan(got)
    assert got["header"][0] == WORKERS and min(per_worker) > 0


def test_entry_plan_at_the_sequence_limit(backend, gpu_device):
    """The entry split's plan (8 kv heads) for NKV_MAX_PLAN_SEQS sequences,
    lengths 0 .. 3000 over 16-row blocks (entries of
    nkv_attention_entry_rows(16) rows, 768 by default): the plan kernel's
    LDS scan at its largest; the whole plan equals the restatement, padding
    entries empty."""
    from nanokv import _lib

    rng = np.random.default_rng(81)
    lens = rng.integers(0, 3001, 8192)
    lens[:7] = [0, 768, 769, 767, 1, 1536, 0]
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)).to(gpu_device)
    cache = torch.empty((1, 16, 8, 128), dtype=torch.bfloat16, device=gpu_device)
    plan, first = backend.build_attention_plan(cache, cu, int(lens.sum()))
    check_entry_plan(plan, first, lens.tolist(), int(_lib.load_library().nkv_attention_entry_rows(16)))


@pytest.mark.parametrize("hkv,g,bs,profile", [
    (2, 8, 16, "short"), (1, 12, 16, "short"), (4, 2, 256, "short"), (2, 16, 32, "mixed"),
    (2, 8, 16, "mixed"), (1, 4, 1, "long")])
def test_workers_span_many_sequences(backend, gpu_device, hkv, g, bs, profile):
    """Splits whose ranges cross many sequence boundaries: 2000 contexts of
    0-48 rows ("short": each worker starts several sequences, many of one
    chunk, so a sequence's q is fetched after its first chunk is already
    in flight; 12 and 16 query heads load q without the prefetch), long
    contexts among short ones ("mixed": ranges inside one context next to
    ranges over dozens), and 8 contexts of 40,000 one-row blocks ("long":
    each range spans hundreds of blocks, past the 64 block ids a worker
    holds at a time)."""
    rng = np.random.default_rng(hkv * 1000 + g * 10 + bs)
    if profile == "short":
        lens = rng.integers(0, 49, 2000)
        lens[rng.random(2000) < 0.2] = 0
    elif profile == "mixed":
        lens = rng.integers(0, 40, 600)
        lens[rng.choice(600, 6, replace=False)] = rng.integers(5000, 20000, 6)
    else:
        lens = np.full(8, 40000)
    lens = lens.tolist()
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv * 7 + g + bs)
    plan, first = backend.build_attention_plan(dev["kc"], dev["cu"], total)
    walk_attention_plan(read_attention_plan(plan, first, len(lens)))
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, scale, plan=(plan, first))
    check_close(out, reference(host, scale), f"{profile} hkv={hkv} g={g} bs={bs}")
    empty = torch.from_numpy(np.asarray(lens) == 0).to(gpu_device)
    assert torch.all(out[empty] == 0), "an empty context must give zeros"


@pytest.mark.parametrize("hkv,g", [(3, 4), (5, 3), (6, 4), (12, 1), (10, 1)])
def test_head_rotation_over_many_entries(backend, gpu_device, hkv, g):
    """Both kernels rotate the kv head over the XCDs: the range kernel with
    the worker (period 32 / gcd(Hkv, 32): 32 for 3 and 5 kv heads, 16 for
    6), the entry kernel with the entry (period 8 / gcd(Hkv, 8): 2 for 12
    and 4 for 10 kv heads); over 40 sequences of up to 2304 rows every
    (worker or entry, head) pair must still be computed exactly once."""
    rng = np.random.default_rng(hkv * 10 + g)
    lens = rng.integers(1, 3 * 768 + 1, 40).tolist()
    dev, host, total = build_case(gpu_device, hkv, g, 16, lens, seed=hkv * 31 + g)
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, scale)
    check_close(out, reference(host, scale), f"rotation hkv={hkv} g={g}")


@pytest.mark.parametrize("hkv,g", [(8, 2), (2, 8)])
def test_invalid_block_ids_drop_their_rows(backend, gpu_device, hkv, g):
    """A block id outside [0, num_blocks) (or -1) inside a context drops that
    block's rows, so the result equals attention over the remaining rows;
    the kernel never reads outside the cache."""
    bs = 16
    lens = [5 * bs, 3 * bs + 4, 2 * bs]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=11)
    nb = host["kc"].shape[0]
    bad_tables = host["tables"].copy()
    bad_tables[0, 2] = nb + 7      # out of range
    bad_tables[1, 0] = -1          # negative
    bad_tables[2, 1] = 2 ** 30     # far out of range
    dev_tables = torch.from_numpy(bad_tables).to(gpu_device)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev_tables, dev["cu"],
                                         total, 1 / math.sqrt(128))
    # expected: the same contexts without the dropped (full) blocks
    kept_tables = np.full_like(host["tables"], -1)
    kept_lens = []
    for i, n in enumerate(lens):
        nblk = -(-n // bs)
        keep = [host["tables"][i, j] for j in range(nblk) if 0 <= bad_tables[i, j] < nb]
        kept_tables[i, : len(keep)] = keep
        kept_lens.append(n - (nblk - len(keep)) * bs)
    ref = reference(dict(host, tables=kept_tables, lens=np.asarray(kept_lens)), 1 / math.sqrt(128))
    check_close(out, ref, "invalid blocks")


@pytest.mark.parametrize("hkv,g", [(8, 2), (2, 1), (1, 2), (2, 8), (4, 4)])
def test_rows_outside_the_contexts_may_hold_any_bits(backend, gpu_device, hkv,
                                                     g):
    """Cache rows no context owns may hold any bits (a cache from torch.empty,
    freed blocks): here NaN and +-Inf in block 0 (which no table uses), in
    the spare blocks and in the unwritten tail of every context's last
    block.  The kernel reads such rows only as masked rows (score -inf, V
    row zeroed), so the result is the oracle's, finite."""
    bs = 16
    lens = [1, 5, bs, 3 * bs + 7, 40, 2, 0]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv * 31 + g)
    nan, inf = float("nan"), float("inf")
    kc = torch.cat([torch.full_like(dev["kc"][:1], nan), dev["kc"]])
    vc = torch.cat([torch.full_like(dev["vc"][:1], inf), dev["vc"]])
    tables = torch.where(dev["tables"] >= 0, dev["tables"] + 1, dev["tables"])
    for i, n in enumerate(lens):
        if n == 0:
            continue
        last = int(host["tables"][i, (n - 1) // bs]) + 1
        tail = n - (n - 1) // bs * bs
        kc[last, tail:] = nan
        vc[last, tail:] = -inf
    used = set(host["tables"][host["tables"] >= 0].tolist())
    for b in range(dev["kc"].shape[0]):
        if b not in used:
            kc[b + 1] = inf
            vc[b + 1] = nan
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_decode(dev["q"], kc, vc, tables, dev["cu"], total, scale)
    assert torch.isfinite(out).all(), "a skipped row reached the sums"
    check_close(out, reference(host, scale), f"any-bits rows hkv={hkv} g={g}")


@pytest.mark.parametrize("hkv,g", [(8, 2), (8, 4), (2, 8), (4, 4)])
def test_cache_over_4gib(backend, gpu_device, hkv, g):
    """Caches larger than 4 GiB, whose row byte offsets need more than 32
    bits (the 64-bit-address instances of the entry kernel, 8 kv heads, and
    of the range kernel, 2 and 4): the contexts' blocks are moved to the
    top of each cache."""
    bs = 256
    lens = [300, 700, 1, 513]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=43)
    compact = dev["kc"].shape[0]
    big = (1 << 32) // (bs * hkv * 128 * 2) + 8  # 4 GiB + 8 blocks per cache
    shift = big - compact
    kc = torch.empty((big, bs, hkv, 128), dtype=torch.bfloat16, device=gpu_device)
    vc = torch.empty_like(kc)
    try:
        kc[:shift].zero_()
        vc[:shift].zero_()
        kc[shift:] = dev["kc"]
        vc[shift:] = dev["vc"]
        tables = torch.where(dev["tables"] >= 0, dev["tables"] + shift, dev["tables"])
        scale = 1.0 / math.sqrt(128)
        out = backend.paged_attention_decode(dev["q"], kc, vc, tables, dev["cu"], total, scale)
        check_close(out, reference(host, scale), f"cache over 4 GiB hkv={hkv} g={g}")
    finally:
        del kc, vc
        torch.cuda.empty_cache()


@pytest.mark.parametrize("hq", [16, 32])
def test_decode_step_layer_full_size(backend, gpu_device, hq):
    """One layer of the 256-sequence decode step (contexts log-uniform in
    [256, 16384], 8 kv heads x 2 or 4 query heads each), every element
    checked."""
    from nanokv import workloads

    wl = workloads.build("decode_step", num_layers=1)
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    gen = torch.Generator(device=gpu_device).manual_seed(3)
    kc = torch.randn(shape, device=gpu_device, generator=gen).to(torch.bfloat16)
    vc = torch.randn(shape, device=gpu_device, generator=gen).to(torch.bfloat16)
    q = torch.randn((wl.num_seqs, hq, 128), device=gpu_device, generator=gen).to(torch.bfloat16)
    tables = wl.padded_block_tables()
    cu = wl.cu_seqlens_k()
    total = int(cu[-1])
    out = backend.paged_attention_decode(q, kc, vc, torch.from_numpy(tables).to(gpu_device),
                                         torch.from_numpy(cu).to(gpu_device), total, 1 / math.sqrt(128))
    torch.cuda.synchronize()
    used = np.unique(tables[tables >= 0])
    remap = np.full(wl.num_blocks, -1, np.int64)
    remap[used] = np.arange(used.size)
    index = torch.from_numpy(used.astype(np.int64)).to(gpu_device)
    hk = kc.index_select(0, index).cpu().view(torch.int16).numpy()
    hv = vc.index_select(0, index).cpu().view(torch.int16).numpy()
    ctables = np.where(tables >= 0, remap[np.maximum(tables, 0)], -1).astype(np.int32)
    ref = reference(dict(q=q.float().cpu().numpy(), kc=hk, vc=hv, tables=ctables,
                         lens=wl.num_tokens), 1 / math.sqrt(128))
    check_close(out, ref, f"decode step layer, {hq} query heads")
