"""Paged-attention decode on the GPU vs the float32 oracle
(oracle.paged_kv.paged_attention_decode, itself pinned to torch's SDPA with
GQA in tests/test_attention_oracle.py).

Two kernels serve the call: the MFMA kernel, the default for every layout
(1-16 query heads per kv head, any kv-head count), and the VALU kernel,
which runs 1-2 query heads per kv head over 1, 2, 4 or 8 kv heads when
NKV_DECODE_VALU=1 is set; the tests marked "valu" set it.  Scores and the
softmax run in fp32 in both; the MFMA kernel rounds the weights p to bf16 /
fp16 before the second product (as flash attention does), and both round
the result once.  Each
rounding is <= 2^-9 relative, so an element differs from the fp32 result by
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

VALU_KV_HEADS = (1, 2, 4, 8)


def with_kernels(layouts):
    """(kernel, *layout) cases: "mfma" for every layout, "valu" as well for
    the layouts the VALU kernel has (1-2 query heads over 1, 2, 4 or 8 kv
    heads)."""
    cases = []
    for layout in layouts:
        cases.append(("mfma", *layout))
        if layout[1] <= 2 and layout[0] in VALU_KV_HEADS:
            cases.append(("valu", *layout))
    return cases


def select_kernel(monkeypatch, kernel: str) -> None:
    """The library reads NKV_DECODE_VALU on every call."""
    if kernel == "valu":
        monkeypatch.setenv("NKV_DECODE_VALU", "1")
    else:
        monkeypatch.delenv("NKV_DECODE_VALU", raising=False)

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


@pytest.mark.parametrize("kernel,hkv,g,bs", with_kernels([
    (8, 2, 256), (8, 2, 16), (2, 8, 256), (2, 8, 16), (4, 4, 16), (4, 2, 32),
    (8, 1, 16), (2, 1, 16), (1, 8, 16), (1, 1, 4), (2, 4, 8),
    (8, 2, 24), (2, 4, 1000),  # block sizes that are not powers of two (1000: entries of 500 rows)
    (8, 4, 16), (4, 7, 256), (4, 8, 16), (8, 3, 16), (2, 5, 8), (1, 6, 16),  # up to 32 query heads
    (8, 5, 16), (8, 8, 256),  # 40 and 64 query heads
    (2, 16, 16), (1, 12, 256), (4, 10, 24), (2, 9, 8),  # 9-16 query heads per kv head
    (3, 4, 16), (16, 2, 16), (6, 1, 32), (5, 3, 256),  # kv-head counts other than 1, 2, 4, 8
]))
def test_decode_attention_matches_oracle(backend, gpu_device, monkeypatch, kernel, hkv, g, bs):
    select_kernel(monkeypatch, kernel)
    lens = [0, 1, bs - 1, bs, bs + 1, 3 * bs + 7, 2, 5 * bs, 17, 1]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv * 100 + g * 10 + bs)
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, scale)
    ref = reference(host, scale)
    check_close(out, ref, f"hkv={hkv} g={g} bs={bs}")
    assert torch.all(out[0] == 0), "an empty context must give zeros"


@pytest.mark.parametrize("kernel,hkv,g,bs", with_kernels([
    (8, 2, 16), (2, 8, 256), (1, 1, 4), (4, 2, 24), (8, 6, 16), (2, 16, 16), (3, 4, 24)]))
def test_decode_attention_float16_matches_oracle(backend, gpu_device, monkeypatch, kernel, hkv, g,
                                                 bs):
    """float16 q and caches (the fp16 MFMAs, or v_dot2 on fp16 pairs), fp16
    output; the same tolerance holds (fp16 rounds to 2^-11)."""
    select_kernel(monkeypatch, kernel)
    lens = [0, 1, bs - 1, bs, bs + 1, 3 * bs + 7, 2, 5 * bs, 17, 1]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv + g + bs,
                                  dtype=torch.float16)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, 0.0884)
    assert out.dtype == torch.float16
    ref = reference(host, 0.0884, "float16")
    check_close(out, ref, f"fp16 hkv={hkv} g={g} bs={bs}")


@pytest.mark.parametrize("kernel,hkv,g", with_kernels([(8, 2), (2, 8)]))
def test_strided_q_plan_reuse_and_out_buffer(backend, gpu_device, monkeypatch, kernel, hkv, g):
    """q with padding heads (row stride past Hq * 128), one plan reused by
    two calls, and a caller-owned output buffer."""
    select_kernel(monkeypatch, kernel)
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


@pytest.mark.parametrize("kernel,hkv,g,bs", with_kernels([
    (8, 2, 16), (2, 4, 8), (4, 2, 4), (1, 1, 1024), (8, 4, 4), (2, 8, 1024)]))
def test_long_contexts_over_small_blocks(backend, gpu_device, monkeypatch, kernel, hkv, g, bs):
    """Entries span many blocks (512 rows of 8- or 16-row blocks, 256 rows =
    64 blocks of 4 rows) or half of one (1024-row blocks); contexts of
    several entries with ragged tails; the plan's entries tile each context
    in order."""
    select_kernel(monkeypatch, kernel)
    from nanokv import _lib

    rows = int(_lib.load_library().nkv_attention_entry_rows(bs))
    lens = [3 * rows + 5, rows, rows + 1, 2 * rows - 1, 7, 1]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv * 7 + g + bs)
    plan, first = backend.build_attention_plan(dev["kc"], dev["cu"], total)
    expect_entries = [-(-n // rows) for n in lens]
    assert first.cpu().tolist() == [0] + np.cumsum(expect_entries).tolist()
    entries = plan.cpu().numpy()[: sum(expect_entries)]
    for i, n in enumerate(lens):
        own = entries[entries[:, 2] == i]
        assert own[:, 0].tolist() == list(range(0, n, rows))
        assert int(own[:, 1].sum()) == n
    assert not plan.cpu().numpy()[sum(expect_entries):, 1].any()  # entries past the total are empty
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, 1 / math.sqrt(128), plan=(plan, first))
    ref = reference(host, 1 / math.sqrt(128))
    check_close(out, ref, f"hkv={hkv} g={g} bs={bs}")


def expected_attention_plan(lens, rows):
    """The decode plan restated: sequence by sequence, entries of `rows`
    context rows in row order (the last one short when rows does not divide
    the length), {row0, rows, seq, 0}; first part of each sequence."""
    first = np.concatenate([[0], np.cumsum([-(-n // rows) for n in lens])]).astype(np.int64)
    entries = [(r, min(rows, n - r), i, 0) for i, n in enumerate(lens) for r in range(0, n, rows)]
    return np.array(entries, dtype=np.int64).reshape(-1, 4), first


def test_plan_at_the_sequence_limit(backend, gpu_device):
    """NKV_MAX_PLAN_SEQS (8192) sequences, lengths 0 .. 3000 over 16-row
    blocks (entries of nkv_attention_entry_rows(16) rows, 768 by default):
    the plan kernel's LDS scan at its largest; the whole plan equals the
    restatement, padding entries empty."""
    from nanokv import _lib

    rng = np.random.default_rng(81)
    lens = rng.integers(0, 3001, 8192)
    lens[:7] = [0, 768, 769, 767, 1, 1536, 0]
    cu = torch.from_numpy(np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)).to(gpu_device)
    cache = torch.empty((1, 16, 1, 128), dtype=torch.bfloat16, device=gpu_device)
    rows = int(_lib.load_library().nkv_attention_entry_rows(16))
    plan, first = backend.build_attention_plan(cache, cu, int(lens.sum()))
    expect, expect_first = expected_attention_plan(lens.tolist(), rows)
    got = plan.cpu().numpy().astype(np.int64)
    np.testing.assert_array_equal(first.cpu().numpy(), expect_first)
    np.testing.assert_array_equal(got[: len(expect)], expect)
    assert not got[len(expect):].any()


@pytest.mark.parametrize("hkv,g", [(3, 4), (5, 3), (6, 4)])
def test_head_rotation_over_many_entries(backend, gpu_device, hkv, g):
    """The MFMA kernel rotates the kv head with the plan entry (period
    8 / gcd(Hkv, 8): 8 for 3 and 5 kv heads, 4 for 6), so each of the 8
    XCDs walks every head; over 40 sequences of up to three 768-row entries
    every (entry, head) pair must still be computed exactly once."""
    rng = np.random.default_rng(hkv * 10 + g)
    lens = rng.integers(1, 3 * 768 + 1, 40).tolist()
    dev, host, total = build_case(gpu_device, hkv, g, 16, lens, seed=hkv * 31 + g)
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, scale)
    check_close(out, reference(host, scale), f"rotation hkv={hkv} g={g}")


@pytest.mark.parametrize("kernel,hkv,g", with_kernels([(8, 2), (2, 8)]))
def test_invalid_block_ids_drop_their_rows(backend, gpu_device, monkeypatch, kernel, hkv, g):
    """A block id outside [0, num_blocks) (or -1) inside a context drops that
    block's rows, so the result equals attention over the remaining rows;
    the kernel never reads outside the cache."""
    select_kernel(monkeypatch, kernel)
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


@pytest.mark.parametrize("kernel,hkv,g", with_kernels([(8, 2), (2, 1), (1, 2), (2, 8), (4, 4)]))
def test_rows_outside_the_contexts_may_hold_any_bits(backend, gpu_device, monkeypatch, kernel, hkv,
                                                     g):
    """Cache rows no context owns may hold any bits (a cache from torch.empty,
    freed blocks): here NaN and +-Inf in block 0 (which no table uses), in
    the spare blocks and in the unwritten tail of every context's last
    block.  The kernels read such rows only as skipped rows, so the result
    is the oracle's, finite, for the MFMA kernel and the VALU kernel (2 x 1
    and 1 x 2 give it 2 and 4 rows per wavefront load)."""
    select_kernel(monkeypatch, kernel)
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


@pytest.mark.parametrize("kernel,hkv,g", with_kernels([(8, 2), (8, 4)]))
def test_cache_over_4gib(backend, gpu_device, monkeypatch, kernel, hkv, g):
    """Caches larger than 4 GiB, whose row byte offsets need more than 32
    bits (the MFMA kernel's 64-bit-address instance; the VALU kernel always
    forms 64-bit offsets): the contexts' blocks are moved to the top of each
    cache."""
    select_kernel(monkeypatch, kernel)
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


@pytest.mark.parametrize("kernel,hq", [("mfma", 16), ("valu", 16), ("mfma", 32)])
def test_decode_step_layer_full_size(backend, gpu_device, monkeypatch, kernel, hq):
    """One layer of the 256-sequence decode step (contexts log-uniform in
    [256, 16384], 8 kv heads x 2 or 4 query heads each), every element
    checked; 2 query heads per kv head on both kernels."""
    select_kernel(monkeypatch, kernel)
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
