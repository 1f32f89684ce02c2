"""Paged-attention prefill on the GPU vs the float32 oracle
(oracle.paged_kv.paged_attention_prefill, pinned to torch's SDPA with the
reference's prefix-causal mask in tests/test_prefill_oracle.py).

Tolerance: scores and the softmax run in fp32; the weights p are rounded to
bf16 before the second product (as flash attention does) and the result to
bf16 once.  Each rounding is <= 2^-9 relative, so an element differs from
the fp32 result by at most 2^-9 * sum_k p_k |v_k| / sum_k p_k (the same
attention over |V|, "ref_abs") plus 2^-9 * |ref|; the tests allow
1e-3 + 2^-8 * (ref_abs + |ref|).  Which keys each query sees is checked
exactly by test_visibility_is_exact (uniform weights, indicator values).
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


def check_close(got: torch.Tensor, ref: np.ndarray, ref_abs: np.ndarray, what: str) -> None:
    g = got.float().cpu().numpy()
    bad = np.abs(g - ref) > ATOL + 2.0 ** -8 * (ref_abs + np.abs(ref))
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {np.abs(g - ref).max():.3e}"


def build_case(device, hkv, g, bs, q_lens, k_lens, seed, q_extra_heads=0, spare_blocks=5,
               dtype=torch.bfloat16):
    gen = torch.Generator().manual_seed(seed)
    b = len(q_lens)
    need = [-(-int(n) // bs) for n in k_lens]
    nb = sum(need) + spare_blocks
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
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    q_full = torch.randn(int(cu_q[-1]), hq + q_extra_heads, 128, generator=gen).to(dtype)
    dev = dict(
        kc=kc.to(device), vc=vc.to(device), q=q_full.to(device)[:, :hq],
        tables=torch.from_numpy(tables).to(device), cu_q=torch.from_numpy(cu_q).to(device),
        cu_k=torch.from_numpy(cu_k).to(device),
    )
    host = dict(q=q_full[:, :hq].float().numpy(), kc=kc.view(torch.int16).numpy(),
                vc=vc.view(torch.int16).numpy(), tables=tables, cu_q=cu_q, cu_k=cu_k,
                dtype=str(dtype).removeprefix("torch."))
    return dev, host


def run(backend, dev, scale, **kw):
    return backend.paged_attention_prefill(dev["q"], dev["kc"], dev["vc"], dev["tables"],
                                           dev["cu_q"], dev["cu_k"], scale, **kw)


def reference(host, scale, tables=None):
    """(fp32 attention, the same attention over |V|)."""
    tables = host["tables"] if tables is None else tables
    ref = oracle.paged_attention_prefill(host["q"], host["cu_q"], host["kc"], host["vc"], tables,
                                         host["cu_k"], scale, dtype=host["dtype"])
    v_abs = host["vc"] & np.int16(0x7FFF)  # bf16 / fp16 words with the sign cleared
    ref_abs = oracle.paged_attention_prefill(host["q"], host["cu_q"], host["kc"], v_abs, tables,
                                             host["cu_k"], scale, dtype=host["dtype"])
    return ref, ref_abs


@pytest.mark.parametrize("hkv,g,bs", [
    (8, 2, 256), (8, 2, 16), (2, 8, 16), (4, 4, 32), (1, 1, 16), (2, 4, 8), (8, 1, 256), (1, 8, 64),
    (16, 1, 16), (3, 2, 16), (6, 1, 32),
    (8, 2, 24), (4, 2, 100),  # block sizes that are not powers of two
    (4, 7, 16), (8, 4, 256), (8, 3, 32), (2, 5, 16), (1, 6, 64),  # Qwen2.5-VL-7B, Qwen3-VL-8B, ...
])
def test_prefill_matches_oracle(backend, gpu_device, hkv, g, bs):
    """Full prompts (Lq == Lk), continuation chunks over a cached prefix
    (Lk > Lq), single-token chunks, chunks of several query tiles, ragged
    last blocks, and an empty request.  Block sizes of 24 and 100 take the
    division path of the row map (the others shift).  Query heads per kv
    head from 1 to 8; with 3, 5, 6 or 7 the last rows of each workgroup
    idle.  The kv head counts
    cover each mapping of workgroups to XCDs: multiples of 8 (8, 16),
    divisors of 8 (1, 2, 4; the plan's length is not a multiple of 8 / H)
    and neither (3, 6)."""
    q_lens = [1, 37, 200, 64, 1, 0, 130]
    k_lens = [1, 37, 333, 64 + 3 * bs + 5, 90, 12, 130]
    dev, host = build_case(gpu_device, hkv, g, bs, q_lens, k_lens, seed=hkv * 100 + g * 10 + bs)
    scale = 1.0 / math.sqrt(128)
    out = run(backend, dev, scale)
    check_close(out, *reference(host, scale), f"hkv={hkv} g={g} bs={bs}")


def check_plan(plan, q_lens, k_lens, tile, longest_first):
    """Every query tile exactly once, entries past the tiles empty, and the
    order: most visible keys first (ties in sequence order, each sequence's
    last tile first), or, for plans too long to sort, sequence by sequence,
    last tile first."""
    total = sum(-(-n // tile) for n in q_lens)
    entries = plan[:total]
    got = sorted((int(s), int(t0), int(n)) for s, t0, n, _ in entries)
    want = sorted((i, t0, min(tile, n - t0)) for i, n in enumerate(q_lens) for t0 in range(0, n, tile))
    assert got == want
    assert not plan[total:, 2].any()
    order = [(int(s), int(t0)) for s, t0, _, _ in entries]
    by_sequence = [(i, t0) for i, n in enumerate(q_lens) for t0 in reversed(range(0, n, tile))]
    if longest_first:
        visible = [k_lens[s] - q_lens[s] + t0 + int(n) for s, t0, n, _ in entries]
        rank = {key: r for r, key in enumerate(by_sequence)}
        assert order == sorted(order, key=lambda k: (-(k_lens[k[0]] - q_lens[k[0]] + k[1]
                                                       + min(tile, q_lens[k[0]] - k[1])), rank[k]))
        assert visible == sorted(visible, reverse=True)
    else:
        assert order == by_sequence


@pytest.mark.parametrize("hkv,g,bs", [(8, 2, 256), (2, 4, 16), (1, 1, 24)])
def test_prefill_float16_matches_oracle(backend, gpu_device, hkv, g, bs):
    """float16 q and caches: the f16 MFMA, weights rounded to fp16, fp16
    output; the same tolerance holds (fp16 rounds to 2^-11)."""
    q_lens = [1, 37, 200, 64, 0, 130]
    k_lens = [1, 37, 333, 64 + 3 * bs + 5, 12, 130]
    dev, host = build_case(gpu_device, hkv, g, bs, q_lens, k_lens, seed=hkv + g + bs,
                           dtype=torch.float16)
    scale = 1.0 / math.sqrt(128)
    out = run(backend, dev, scale)
    assert out.dtype == torch.float16
    check_close(out, *reference(host, scale), f"fp16 hkv={hkv} g={g} bs={bs}")


def test_plan_tiles_cover_every_query(backend, gpu_device):
    from nanokv import _lib

    q_lens, k_lens = [200, 1, 0, 64, 65], [300, 5, 3, 64, 65]
    dev, host = build_case(gpu_device, 8, 2, 16, q_lens, k_lens, seed=3)
    tile = int(_lib.load_library().nkv_prefill_tile_tokens(2))
    assert tile in (64, 128)  # 128 or 256 query rows per workgroup, 2 heads per token
    plan = backend.build_prefill_plan(dev["q"], dev["kc"], dev["cu_q"], dev["cu_k"]).cpu().numpy()
    check_plan(plan, q_lens, k_lens, tile, longest_first=True)


@pytest.mark.parametrize("num_seqs,mean_tokens", [(37, 300), (700, 900)])
def test_plan_order_at_scale(gpu_device, num_seqs, mean_tokens):
    """Random lengths and cached prefixes: 37 requests (a plan whose length
    is not a power of two, sorted in LDS) and 700 requests at 8 query heads
    per kv head (over 2048 tiles: the unsorted fallback)."""
    from nanokv import _lib
    from nanokv.paged_kv import ops

    rng = np.random.default_rng(num_seqs)
    q_lens = rng.integers(0, 2 * mean_tokens, num_seqs).tolist()
    k_lens = [q + int(c) for q, c in zip(q_lens, rng.integers(0, 3000, num_seqs))]
    group = 2 if num_seqs < 100 else 8
    tile = int(_lib.load_library().nkv_prefill_tile_tokens(group))
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32, device=gpu_device)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(k_lens)]), dtype=torch.int32, device=gpu_device)
    plan = ops.build_prefill_plan(cu_q, cu_k, sum(q_lens), group).cpu().numpy()
    tiles = sum(-(-n // tile) for n in q_lens)
    assert (tiles <= 2048) == (num_seqs < 100)
    check_plan(plan, q_lens, k_lens, tile, longest_first=plan.shape[0] <= 2048)


def test_strided_q_plan_reuse_and_out_buffer(backend, gpu_device):
    """q as a view of a wider projection (token stride > Hq * D), a plan
    built once and reused, and a caller-provided output."""
    q_lens, k_lens = [70, 9], [100, 9]
    dev, host = build_case(gpu_device, 8, 2, 16, q_lens, k_lens, seed=7, q_extra_heads=8)
    assert dev["q"].stride(0) == 24 * 128
    plan = backend.build_prefill_plan(dev["q"], dev["kc"], dev["cu_q"], dev["cu_k"])
    out = torch.empty((sum(q_lens), 16, 128), dtype=torch.bfloat16, device=gpu_device)
    ref, ref_abs = reference(host, 0.1)
    for _ in range(2):
        out.zero_()
        run(backend, dev, 0.1, plan=plan, out=out)
        check_close(out, ref, ref_abs, "planned")


def test_invalid_block_ids_drop_their_keys(backend, gpu_device):
    bs = 16
    q_lens, k_lens = [20, 8], [5 * bs, 3 * bs + 4]
    dev, host = build_case(gpu_device, 4, 2, bs, q_lens, k_lens, seed=11)
    nb = host["kc"].shape[0]
    bad = host["tables"].copy()
    bad[0, 1] = nb + 7   # a prefix block out of range
    bad[1, 0] = -1       # negative
    out = backend.paged_attention_prefill(dev["q"], dev["kc"], dev["vc"],
                                          torch.from_numpy(bad).to(gpu_device), dev["cu_q"],
                                          dev["cu_k"], 1 / math.sqrt(128))
    # expected: the same keys without the dropped blocks, positions unchanged
    ref = np.zeros((sum(q_lens), 8, 128), np.float32)
    ref_abs = np.zeros_like(ref)
    k = [oracle.bf16_words_to_f32(oracle.gather(host["kc"], host["tables"][i], n)) for i, n in enumerate(k_lens)]
    v = [oracle.bf16_words_to_f32(oracle.gather(host["vc"], host["tables"][i], n)) for i, n in enumerate(k_lens)]
    scale = 1 / math.sqrt(128)
    for i, (lq, lk) in enumerate(zip(q_lens, k_lens)):
        kept = np.array([0 <= bad[i, t // bs] < nb for t in range(lk)])
        for j in range(lq):
            visible = kept & (np.arange(lk) <= lk - lq + j)
            for h in range(8):
                if not visible.any():
                    continue
                s = (k[i][visible, h // 2] @ host["q"][host["cu_q"][i] + j, h]) * scale
                p = np.exp(s - s.max())
                ref[host["cu_q"][i] + j, h] = (p / p.sum()) @ v[i][visible, h // 2]
                ref_abs[host["cu_q"][i] + j, h] = (p / p.sum()) @ np.abs(v[i][visible, h // 2])
    check_close(out, ref, ref_abs, "invalid blocks")


@pytest.mark.parametrize("g,bs", [(2, 16), (1, 256), (8, 8)])
def test_visibility_is_exact(backend, gpu_device, g, bs):
    """q = 0 makes every visible key weigh exactly 1 (also after bf16
    rounding), and V[t][d] = 1 when t % 128 == d, else 0: output[j][d] is
    then the count of visible keys t with t % 128 == d over the count of
    visible keys, which is exact in fp32.  Any key wrongly shown or hidden
    (tile boundaries, the causal offset, ragged blocks) moves some element
    by far more than the bf16 rounding of the result."""
    q_lens = [1, 70, 130, 5]
    k_lens = [1, 70, 300, 200]
    hkv = 2
    dev, host = build_case(gpu_device, hkv, g, bs, q_lens, k_lens, seed=5)
    nb = host["kc"].shape[0]
    vc = torch.zeros((nb, bs, hkv, 128), dtype=torch.bfloat16)
    for i, lk in enumerate(k_lens):
        for t in range(lk):
            vc[host["tables"][i, t // bs], t % bs, :, t % 128] = 1.0
    q0 = torch.zeros_like(dev["q"])
    out = backend.paged_attention_prefill(q0, dev["kc"], vc.to(gpu_device), dev["tables"],
                                          dev["cu_q"], dev["cu_k"], 0.7).float().cpu().numpy()
    for i, (lq, lk) in enumerate(zip(q_lens, k_lens)):
        for j in range(lq):
            n = lk - lq + j + 1  # keys 0 .. n-1 visible
            expect = np.array([len(range(d, n, 128)) for d in range(128)], np.float32) / n
            got = out[host["cu_q"][i] + j]
            np.testing.assert_allclose(got, np.broadcast_to(expect, got.shape), rtol=2.0 ** -8,
                                       atol=0, err_msg=f"request {i} query {j}")


def test_cache_over_4gib(backend, gpu_device):
    """Caches larger than 4 GiB, whose row byte offsets need more than 32
    bits: the requests' blocks are moved to the top of each cache."""
    hkv, g, bs = 8, 2, 256
    q_lens, k_lens = [70, 5, 130], [300, 700, 130]
    dev, host = build_case(gpu_device, hkv, g, bs, q_lens, k_lens, seed=41, spare_blocks=0)
    compact = dev["kc"].shape[0]
    big = (1 << 32) // (bs * hkv * 128 * 2) + 8  # 4 GiB + 8 blocks per cache
    shift = big - compact
    kc = torch.empty((big, bs, hkv, 128), dtype=torch.bfloat16, device=gpu_device)
    vc = torch.empty_like(kc)
    try:
        kc[shift:] = dev["kc"]
        vc[shift:] = dev["vc"]
        tables = torch.where(dev["tables"] >= 0, dev["tables"] + shift, dev["tables"])
        scale = 1.0 / math.sqrt(128)
        out = backend.paged_attention_prefill(dev["q"], kc, vc, tables, dev["cu_q"], dev["cu_k"],
                                              scale)
        check_close(out, *reference(host, scale), "cache over 4 GiB")
    finally:
        del kc, vc
        torch.cuda.empty_cache()


@pytest.mark.parametrize("hkv,g", [(8, 2), (2, 8)])
def test_rows_outside_the_contexts_may_hold_any_bits(backend, gpu_device, hkv, g):
    """Cache rows no context owns may hold any bits: NaN and +-Inf in block 0
    (which no table uses), in the spare blocks and in the unwritten tail of
    every context's last block.  The result is the oracle's, finite."""
    bs = 16
    q_lens, k_lens = [5, 1, 40, 16], [5, 33, 70, 16]
    dev, host = build_case(gpu_device, hkv, g, bs, q_lens, k_lens, seed=hkv * 17 + g)
    nan, inf = float("nan"), float("inf")
    kc = torch.cat([torch.full_like(dev["kc"][:1], nan), dev["kc"]])
    vc = torch.cat([torch.full_like(dev["vc"][:1], -inf), dev["vc"]])
    tables = torch.where(dev["tables"] >= 0, dev["tables"] + 1, dev["tables"])
    for i, n in enumerate(k_lens):
        last = int(host["tables"][i, (n - 1) // bs]) + 1
        tail = n - (n - 1) // bs * bs
        kc[last, tail:] = inf
        vc[last, tail:] = nan
    used = set(host["tables"][host["tables"] >= 0].tolist())
    for b in range(dev["kc"].shape[0]):
        if b not in used:
            kc[b + 1] = nan
            vc[b + 1] = inf
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_prefill(dev["q"], kc, vc, tables, dev["cu_q"], dev["cu_k"], scale)
    assert torch.isfinite(out).all(), "a row outside the contexts reached the sums"
    check_close(out, *reference(host, scale), f"any-bits rows hkv={hkv} g={g}")


def test_unsupported_layouts_raise(backend, gpu_device):
    dev, _ = build_case(gpu_device, 3, 1, 16, [4], [4], seed=1)
    q9 = torch.zeros((4, 27, 128), dtype=torch.bfloat16, device=gpu_device)  # G = 9
    with pytest.raises((ValueError, RuntimeError)):
        backend.paged_attention_prefill(q9, dev["kc"], dev["vc"], dev["tables"], dev["cu_q"],
                                        dev["cu_k"], 0.1)


def test_plan_for_another_head_layout_is_rejected(backend, gpu_device):
    """A plan built for one query head per kv head has 128-token tiles; the
    two-heads-per-kv-head kernel takes 64-token tiles, so reusing it would
    leave queries out.  Its size gives it away."""
    q_lens, k_lens = [300, 40], [300, 90]
    dev, _ = build_case(gpu_device, 8, 2, 16, q_lens, k_lens, seed=13)
    q1 = dev["q"][:, :8]  # one query head per kv head
    plan1 = backend.build_prefill_plan(q1, dev["kc"], dev["cu_q"], dev["cu_k"])
    with pytest.raises(ValueError, match="prefill plan"):
        run(backend, dev, 0.1, plan=plan1)


def test_chunked_prefill_full_size(backend, gpu_device):
    """The chunked-prefill step at full size: 16 requests in one 8192-token
    chunk (lengths uniform in [128, 4096] scaled to the chunk), requests 0-7
    continuing after 1-4 cached blocks; 8 kv heads x 2 query heads each,
    256-row blocks.  Every element is checked against the oracle."""
    rng = np.random.default_rng(17)
    raw = rng.integers(128, 4097, 16).astype(np.float64)
    q_lens = np.floor(raw / raw.sum() * 8192).astype(np.int64)
    q_lens[-1] += 8192 - q_lens.sum()
    cached = np.zeros(16, np.int64)
    cached[:8] = rng.integers(1, 5, 8) * 256
    k_lens = q_lens + cached
    dev, host = build_case(gpu_device, 8, 2, 256, q_lens.tolist(), k_lens.tolist(), seed=29)
    scale = 1 / math.sqrt(128)
    out = run(backend, dev, scale)
    check_close(out, *reference(host, scale), "chunked prefill")


# ------------------------------------------------ flash-attn call drop-ins

def test_flash_varlen_with_block_table_matches_oracle(gpu_device):
    """attention.py:105-116: flash_attn_varlen_func(q, k_cache, v_cache,
    ..., causal=True, block_table=...)."""
    from nanokv.flash import flash_attn_varlen_func

    q_lens, k_lens = [37, 1, 130], [300, 9, 130]
    dev, host = build_case(gpu_device, 8, 2, 16, q_lens, k_lens, seed=23)
    out = flash_attn_varlen_func(dev["q"], dev["kc"], dev["vc"], max_seqlen_q=max(q_lens),
                                 cu_seqlens_q=dev["cu_q"], max_seqlen_k=max(k_lens),
                                 cu_seqlens_k=dev["cu_k"], softmax_scale=0.09, causal=True,
                                 block_table=dev["tables"])
    check_close(out, *reference(host, 0.09), "flash varlen paged")


def test_flash_varlen_contiguous_keys_matches_oracle(gpu_device):
    """The reference's prefill without block tables passes the step's own
    k and v (views of the QKV projection) back to back."""
    from nanokv.flash import flash_attn_varlen_func

    q_lens = [70, 5, 129]
    dev, host = build_case(gpu_device, 4, 2, 16, q_lens, q_lens, seed=31)
    total = sum(q_lens)
    k_rows = np.concatenate([oracle.gather(host["kc"], host["tables"][i], n) for i, n in enumerate(q_lens)])
    v_rows = np.concatenate([oracle.gather(host["vc"], host["tables"][i], n) for i, n in enumerate(q_lens)])
    qkv = torch.zeros((total, 16 * 128), dtype=torch.bfloat16, device=gpu_device)
    k = qkv[:, 8 * 128:12 * 128].view(total, 4, 128)  # strided views, as after the QKV split
    v = qkv[:, 12 * 128:].view(total, 4, 128)
    k.copy_(torch.from_numpy(k_rows).view(torch.bfloat16).to(gpu_device))
    v.copy_(torch.from_numpy(v_rows).view(torch.bfloat16).to(gpu_device))
    out = flash_attn_varlen_func(dev["q"], k, v, max(q_lens), dev["cu_q"], max(q_lens), dev["cu_q"],
                                 softmax_scale=0.1, causal=True)
    check_close(out, *reference(host, 0.1), "flash varlen contiguous")


def check_decode(out, host, lengths, scale, what):
    """Decode output [batch, 1, heads, 128] against the oracle within
    1e-3 + 2^-8 (ref_abs + |ref|), ref_abs being the same attention over |V|
    (the MFMA kernel rounds its weights to the input type, so an output near
    zero by cancellation carries the error of its terms)."""
    args = (host["q"], host["kc"])
    tail = (host["tables"], np.array(lengths), scale)
    ref = oracle.paged_attention_decode(*args, host["vc"], *tail, dtype=host["dtype"])
    ref_abs = oracle.paged_attention_decode(*args, host["vc"] & np.int16(0x7FFF), *tail,
                                            dtype=host["dtype"])
    g = out[:, 0].float().cpu().numpy()
    bad = np.abs(g - ref) > 1e-3 + 2.0 ** -8 * (ref_abs + np.abs(ref))
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {np.abs(g - ref).max():.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_flash_with_kvcache_matches_decode_oracle(gpu_device, dtype):
    """attention.py:122-130: flash_attn_with_kvcache(q.unsqueeze(1), k_cache,
    v_cache, cache_seqlens=context_lens, block_table=..., causal=True), for
    bf16 and fp16 models."""
    from nanokv.flash import flash_attn_with_kvcache

    k_lens = [1, 300, 17, 64]
    dev, host = build_case(gpu_device, 8, 2, 16, [1] * 4, k_lens, seed=37, dtype=dtype)
    lens = torch.tensor(k_lens, dtype=torch.int32, device=gpu_device)
    out = flash_attn_with_kvcache(dev["q"].unsqueeze(1), dev["kc"], dev["vc"], cache_seqlens=lens,
                                  block_table=dev["tables"], softmax_scale=0.088, causal=True)
    assert out.shape == (4, 1, 16, 128) and out.dtype == dtype
    check_decode(out, host, k_lens, 0.088, "flash_attn_with_kvcache")


@pytest.mark.parametrize("hkv,g", [(8, 2), (2, 8)])
def test_flash_with_kvcache_plan_follows_each_step(gpu_device, hkv, g):
    """The decode drop-in builds one plan per step (on its first call, after
    one read of the context total) and reuses it for the step's other
    layers, which pass the same lengths tensor and caches of their own.  It
    must rebuild when the lengths change: an in-place update (torch bumps
    the tensor's version), a new batch packed into the same graph buffers by
    the device packer (which bumps the versions of what its kernel wrote),
    and a layer's cache coming back (the next step).  The longer contexts
    come second, so a stale plan would drop rows and miss the oracle; both
    splits (8 kv heads: entries, 2: ranges)."""
    from nanokv import flash
    from nanokv.packing import DecodeGraphBuffers, DevicePacker, SequenceBatch

    bs = 16
    long_lens = [1, 300, 17, 64]
    dev, host = build_case(gpu_device, hkv, g, bs, [1] * 4, long_lens, seed=53)
    q = dev["q"].unsqueeze(1)
    # three "layers": the same cache contents at three addresses
    layers = [(dev["kc"], dev["vc"])] + [(dev["kc"].clone(), dev["vc"].clone()) for _ in range(2)]

    def run(lengths, tables, layer, lengths_host, what):
        kc, vc = layers[layer]
        out = flash.flash_attn_with_kvcache(q, kc, vc, cache_seqlens=lengths, block_table=tables,
                                            softmax_scale=0.088, causal=True)
        check_decode(out, host, lengths_host, 0.088, what)

    short_lens = [1, 20, 5, 3]
    lens = torch.tensor(short_lens, dtype=torch.int32, device=gpu_device)
    run(lens, dev["tables"], 0, short_lens, "first layer of a step")
    entry = flash._STEP_PLAN._entry
    run(lens, dev["tables"], 1, short_lens, "second layer")
    assert flash._STEP_PLAN._entry is entry, "the step's plan is reused by its next layer"
    lens.copy_(torch.tensor(long_lens, dtype=torch.int32))
    run(lens, dev["tables"], 2, long_lens, "lengths updated in place (version)")
    assert flash._STEP_PLAN._entry is not entry
    entry = flash._STEP_PLAN._entry
    run(lens, dev["tables"], 0, long_lens, "a layer not yet seen with this plan")
    assert flash._STEP_PLAN._entry is entry
    run(lens, dev["tables"], 2, long_lens, "a layer's cache again: the next step")
    assert flash._STEP_PLAN._entry is not entry

    width = host["tables"].shape[1]
    buffers = DecodeGraphBuffers.allocate(gpu_device, max_num_seqs=4, max_blocks=width)
    packer = DevicePacker(gpu_device, bs)

    def pack(lengths_host):
        lists = [host["tables"][i, :-(-n // bs)].tolist() for i, n in enumerate(lengths_host)]
        packer.pack_decode_into(SequenceBatch.from_block_lists(lengths_host, lists), buffers)

    pack(short_lens)
    view = buffers.context_lens  # the same tensor object for both batches
    run(view, buffers.block_tables, 1, short_lens, "first packed batch")
    pack(long_lens)
    run(view, buffers.block_tables, 2, long_lens, "second batch packed into the same buffers")

    # the reference's engine runs under torch.inference_mode(): its lengths
    # carry no version counter, and a step is told by the layers' caches
    with torch.inference_mode():
        lens_inf = torch.tensor(long_lens, dtype=torch.int32, device=gpu_device)
        assert lens_inf.is_inference()
        run(lens_inf, dev["tables"], 0, long_lens, "inference tensor, first layer")
        entry = flash._STEP_PLAN._entry
        run(lens_inf, dev["tables"], 1, long_lens, "inference tensor, second layer")
        assert flash._STEP_PLAN._entry is entry


def test_flash_dropins_reject_what_they_do_not_compute(gpu_device):
    from nanokv.flash import flash_attn_varlen_func, flash_attn_with_kvcache

    dev, _ = build_case(gpu_device, 8, 2, 16, [4], [4], seed=2)
    with pytest.raises(NotImplementedError):
        flash_attn_varlen_func(dev["q"], dev["kc"], dev["vc"], 4, dev["cu_q"], 4, dev["cu_k"],
                               causal=False, block_table=dev["tables"])
    with pytest.raises(NotImplementedError):
        flash_attn_varlen_func(dev["q"], dev["kc"], dev["vc"], 4, dev["cu_q"], 4, dev["cu_k"],
                               causal=True, block_table=dev["tables"], window_size=(8, 0))
    with pytest.raises(TypeError):
        flash_attn_with_kvcache(dev["q"][:1].unsqueeze(1), dev["kc"], dev["vc"],
                                cache_seqlens=dev["cu_k"][1:], block_table=dev["tables"],
                                causal=True, rotary_cos=None)
