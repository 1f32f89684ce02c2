"""HIP backend vs the oracle, bit-exact (integer-word comparison).

Covers the reference's own GPU test matrices (tests/test_paged_kv_cuda.py:
22-46 seed 7, :51-78 fused QKV seed 29, :80-153 full matrix seed 23,
:155-185 native allocation seed 11, :245-273 decode replay), the golden
vectors, edge cases (empty inputs, -1 and out-of-range indices, misaligned
rows) and the five workload shapes at full size.  Every HIP call goes
through the C ABI of libnanokv.so.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle import paged_kv as oracle

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "paged_kv_golden.json").read_text())
WORD = {torch.float16: torch.int16, torch.bfloat16: torch.int16, torch.float32: torch.int32}


def words(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(WORD[t.dtype]).numpy()


@pytest.fixture(scope="module")
def backend(gpu_device):
    from nanokv.paged_kv import create_paged_kv_backend

    return create_paged_kv_backend("hip")


def oracle_store(key, value, kc, vc, slots):
    hk, hv = words(kc).copy(), words(vc).copy()
    oracle.store(words(key), words(value), hk, hv, slots.cpu().numpy())
    return hk, hv


# -------------------------------------------------- reference test matrices

def test_triton_matrix_seed7(backend, gpu_device):
    torch.manual_seed(7)
    for dtype in (torch.float16, torch.bfloat16):
        for heads, head_dim in ((1, 64), (2, 128), (8, 64)):
            key = torch.randn(9, heads, head_dim, device=gpu_device, dtype=dtype)
            value = torch.randn_like(key)
            slots = torch.tensor([0, 17, -1, 4, 31, 8, 23, 2, 15], device=gpu_device, dtype=torch.int32)
            kc = torch.full((4, 8, heads, head_dim), -3, device=gpu_device, dtype=dtype)
            vc = torch.full_like(kc, -3)
            hk, hv = oracle_store(key, value, kc, vc, slots)
            backend.store(key, value, kc, vc, slots)
            np.testing.assert_array_equal(words(kc), hk)
            np.testing.assert_array_equal(words(vc), hv)
            table = torch.tensor([3, 1, 0], device=gpu_device, dtype=torch.int32)
            np.testing.assert_array_equal(
                words(backend.gather(kc, table, 19)), oracle.gather(hk, np.array([3, 1, 0]), 19)
            )


def test_fused_qkv_strided_key_seed29(backend, gpu_device):
    torch.manual_seed(29)
    packed = torch.randn(9, 8, 64, dtype=torch.float16, device=gpu_device)
    key, value = packed[:, 4:6], packed[:, 6:8]
    assert key.stride(0) > key.shape[1] * key.shape[2]
    slots = torch.tensor([0, 17, 4, 31, 8, 23, 2, 15, 9], dtype=torch.int32, device=gpu_device)
    kc = torch.full((4, 8, 2, 64), -3, dtype=torch.float16, device=gpu_device)
    vc = torch.full_like(kc, -3)
    hk, hv = kc.cpu().view(torch.int16).numpy().copy(), vc.cpu().view(torch.int16).numpy().copy()
    c_oracle.store(key.cpu().view(torch.int16).numpy(), value.cpu().view(torch.int16).numpy(), hk, hv,
                   slots.cpu().numpy())
    backend.store(key, value, kc, vc, slots)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(words(kc), hk)
    np.testing.assert_array_equal(words(vc), hv)


def test_registered_ops_dispatch_to_hip(backend, gpu_device):
    """paged_kv.cpp:199-203: callers of torch.ops.nanovllm_paged_kv.store /
    gather / gather_varlen (rather than the backend object) reach the same
    kernels through the schemas registered on the CUDA key."""
    torch.manual_seed(41)
    backend._load()  # loads the library and registers the ops
    key = torch.randn(9, 2, 64, device=gpu_device, dtype=torch.bfloat16)
    value = torch.randn_like(key)
    slots = torch.tensor([0, 17, -1, 4, 31, 8, 23, 2, 15], device=gpu_device, dtype=torch.int32)
    kc = torch.full((4, 8, 2, 64), -3, device=gpu_device, dtype=torch.bfloat16)
    vc = torch.full_like(kc, -3)
    hk, hv = oracle_store(key, value, kc, vc, slots)
    torch.ops.nanovllm_paged_kv.store(key, value, kc, vc, slots)
    np.testing.assert_array_equal(words(kc), hk)
    np.testing.assert_array_equal(words(vc), hv)
    table = torch.tensor([3, 1, 0], device=gpu_device, dtype=torch.int32)
    np.testing.assert_array_equal(words(torch.ops.nanovllm_paged_kv.gather(kc, table, 19)),
                                  oracle.gather(hk, np.array([3, 1, 0]), 19))
    tables = torch.tensor([[3, 1, 0], [2, -1, -1]], device=gpu_device, dtype=torch.int32)
    cu = torch.tensor([0, 19, 24], device=gpu_device, dtype=torch.int32)
    k_out, v_out = torch.ops.nanovllm_paged_kv.gather_varlen(kc, vc, tables, cu, 24)
    expect_k = np.concatenate([oracle.gather(hk, np.array([3, 1, 0]), 19), oracle.gather(hk, np.array([2]), 5)])
    expect_v = np.concatenate([oracle.gather(hv, np.array([3, 1, 0]), 19), oracle.gather(hv, np.array([2]), 5)])
    np.testing.assert_array_equal(words(k_out), expect_k)
    np.testing.assert_array_equal(words(v_out), expect_v)


def test_registered_ops_index_dtype_and_strides(backend, gpu_device):
    """A direct op call (no backend validators in front) with int64 slots or
    block table raises, as the reference op's typed data_ptr<int32_t> does;
    strided int32 index views are read by element, not by raw memory."""
    backend._load()
    torch.manual_seed(43)
    key = torch.randn(6, 2, 64, device=gpu_device, dtype=torch.bfloat16)
    value = torch.randn_like(key)
    kc = torch.full((4, 8, 2, 64), -3, device=gpu_device, dtype=torch.bfloat16)
    vc = torch.full_like(kc, -3)
    with pytest.raises(RuntimeError, match="int32"):
        torch.ops.nanovllm_paged_kv.store(key, value, kc, vc,
                                          torch.arange(6, device=gpu_device, dtype=torch.int64))
    with pytest.raises(RuntimeError, match="int32"):
        torch.ops.nanovllm_paged_kv.gather(kc, torch.tensor([3, 1], device=gpu_device), 9)
    # every other element of a 12-element buffer: slots [5, 30, -1, 9, 2, 17]
    wide = torch.tensor([5, 0, 30, 0, -1, 0, 9, 0, 2, 0, 17, 0], device=gpu_device, dtype=torch.int32)
    slots = wide[::2]
    hk, hv = oracle_store(key, value, kc, vc, slots.contiguous())
    torch.ops.nanovllm_paged_kv.store(key, value, kc, vc, slots)
    np.testing.assert_array_equal(words(kc), hk)
    np.testing.assert_array_equal(words(vc), hv)
    table = torch.tensor([[3, 7], [1, 7], [0, 7]], device=gpu_device, dtype=torch.int32)[:, 0]
    np.testing.assert_array_equal(words(torch.ops.nanovllm_paged_kv.gather(kc, table, 19)),
                                  oracle.gather(hk, np.array([3, 1, 0]), 19))
    # gather_varlen: int64 tables or lengths raise; a column-strided table is read by element
    cu = torch.tensor([0, 19, 24], device=gpu_device, dtype=torch.int32)
    tables = torch.tensor([[3, 1, 0], [2, -1, -1]], device=gpu_device, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="int32"):
        torch.ops.nanovllm_paged_kv.gather_varlen(kc, vc, tables.long(), cu, 24)
    with pytest.raises(RuntimeError, match="int32"):
        torch.ops.nanovllm_paged_kv.gather_varlen(kc, vc, tables, cu.long(), 24)
    strided = torch.stack([tables, torch.full_like(tables, 7)], dim=2).reshape(2, 6)[:, ::2]
    assert strided.stride(1) == 2 and torch.equal(strided, tables)
    k_out, v_out = torch.ops.nanovllm_paged_kv.gather_varlen(kc, vc, strided, cu, 24)
    np.testing.assert_array_equal(words(k_out), np.concatenate(
        [oracle.gather(hk, np.array([3, 1, 0]), 19), oracle.gather(hk, np.array([2]), 5)]))
    np.testing.assert_array_equal(words(v_out), np.concatenate(
        [oracle.gather(hv, np.array([3, 1, 0]), 19), oracle.gather(hv, np.array([2]), 5)]))


def test_store_of_head_strided_views(backend, gpu_device):
    """A view strided between heads (kv[:, :, :128] of a [T, H, 256]
    tensor) passes the validators, which only ask for a contiguous last
    dimension; the store must still copy each head's own 128 elements, as
    the pytorch backend's index_copy_ does."""
    torch.manual_seed(43)
    wide = torch.randn(11, 4, 256, device=gpu_device, dtype=torch.bfloat16)
    key, value = wide[:, :, :128], wide[:, :, 128:]
    assert key.stride(1) == 256 and key.stride(-1) == 1
    slots = torch.tensor([3, -1, 40, 7, 63, 0, 22, 9, 51, -1, 30], dtype=torch.int32, device=gpu_device)
    kc = torch.full((4, 16, 4, 128), -3, device=gpu_device, dtype=torch.bfloat16)
    vc = torch.full_like(kc, -3)
    hk, hv = oracle_store(key.contiguous(), value.contiguous(), kc, vc, slots)
    backend.store(key, value, kc, vc, slots)
    np.testing.assert_array_equal(words(kc), hk)
    np.testing.assert_array_equal(words(vc), hv)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_legacy_store_kvcache_on_fused_qkv(gpu_device, dtype):
    """attention.py:10-33 / :86-93: the layer's fallback store when no
    backend is bound, called with the K/V views of the fused QKV output."""
    from nanokv.paged_kv import store_kvcache

    torch.manual_seed(31)
    heads_q, heads_kv, dim = 8, 2, 128
    qkv = torch.randn(13, (heads_q + 2 * heads_kv) * dim, device=gpu_device, dtype=dtype)
    _, k, v = qkv.split([heads_q * dim, heads_kv * dim, heads_kv * dim], dim=-1)
    k, v = k.view(-1, heads_kv, dim), v.view(-1, heads_kv, dim)
    slots = torch.tensor([5, -1, 0, 63, 17, -1, 40, 2, 33, 48, 9, 61, 26], dtype=torch.int32, device=gpu_device)
    kc = torch.full((4, 16, heads_kv, dim), -3, device=gpu_device, dtype=dtype)
    vc = torch.full_like(kc, -3)
    hk, hv = oracle_store(k, v, kc, vc, slots)
    store_kvcache(k, v, kc, vc, slots)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(words(kc), hk)
    np.testing.assert_array_equal(words(vc), hv)


def test_full_parity_matrix_seed23(backend, gpu_device):
    torch.manual_seed(23)
    num_blocks, block_size = 41, 16
    num_slots = num_blocks * block_size
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        for heads in (1, 2, 8):
            for head_dim in (64, 80, 128, 256):
                for tokens in (1, 8, 257):
                    for mapping in ("contiguous", "random_with_skips"):
                        key = torch.randn(tokens, heads, head_dim, device=gpu_device, dtype=dtype)
                        value = torch.randn_like(key)
                        if mapping == "contiguous":
                            slots = torch.arange(tokens, device=gpu_device, dtype=torch.int32)
                        else:
                            slots = torch.randperm(num_slots, device=gpu_device, dtype=torch.int32)[:tokens]
                            slots[::11] = -1
                        kc = torch.full((num_blocks, block_size, heads, head_dim), -3,
                                        device=gpu_device, dtype=dtype)
                        vc = torch.full_like(kc, -3)
                        hk, hv = oracle_store(key, value, kc, vc, slots)
                        stream = torch.cuda.Stream()
                        stream.wait_stream(torch.cuda.current_stream())
                        with torch.cuda.stream(stream):
                            backend.store(key, value, kc, vc, slots)
                        stream.synchronize()
                        case = f"{dtype} h={heads} d={head_dim} t={tokens} {mapping}"
                        np.testing.assert_array_equal(words(kc), hk, err_msg=case)
                        np.testing.assert_array_equal(words(vc), hv, err_msg=case)
                        table = torch.randperm(num_blocks, device=gpu_device, dtype=torch.int32)
                        length = min(tokens, num_slots)
                        np.testing.assert_array_equal(
                            words(backend.gather(kc, table, length)),
                            oracle.gather(hk, table.cpu().numpy(), length), err_msg=case,
                        )


def test_native_allocation_seed11(backend, gpu_device):
    torch.manual_seed(11)
    allocation = backend.allocate((2, 5, 8, 2, 128), dtype=torch.bfloat16, device="cuda")
    assert allocation.tensor.shape == (2, 5, 8, 2, 128)
    allocation.tensor.fill_(-5)
    kc, vc = allocation.tensor[0], allocation.tensor[1]
    key = torch.randn(10, 2, 128, device=gpu_device, dtype=torch.bfloat16)
    value = torch.randn_like(key)
    slots = torch.tensor([0, 9, 17, -1, 31, 2, 7, 20, 39, 12], device=gpu_device, dtype=torch.int32)
    hk, hv = oracle_store(key, value, kc, vc, slots)
    backend.store(key, value, kc, vc, slots)
    np.testing.assert_array_equal(words(kc), hk)
    np.testing.assert_array_equal(words(vc), hv)
    table = torch.tensor([4, 1, 3], device=gpu_device, dtype=torch.int32)
    np.testing.assert_array_equal(words(backend.gather(kc, table, 19)), oracle.gather(hk, [4, 1, 3], 19))


def test_decode_replay_last_writes_win(backend, gpu_device):
    g = GOLDEN["decode_replay"]
    allocation = backend.allocate((2, *g["cache_shape"]), dtype=torch.float16, device="cuda")
    allocation.tensor.fill_(-1)
    kc, vc = allocation.tensor[0], allocation.tensor[1]
    for step in range(g["steps"]):
        key = torch.full((1, 1, 64), step, dtype=torch.float16, device=gpu_device)
        slot = torch.tensor([step % 16], dtype=torch.int32, device=gpu_device)
        backend.store(key, -key, kc, vc, slot)
    torch.cuda.synchronize()
    assert kc[0, :, 0, 0].cpu().tolist() == [float(v) for v in g["expected_key_column"]]
    assert vc[0, :, 0, 0].cpu().tolist() == [float(v) for v in g["expected_value_column"]]


# ------------------------------------------------------------------ goldens

@pytest.mark.parametrize("case", ["store", "slot_matrix", "native_allocation"])
def test_goldens_on_gpu(backend, gpu_device, case):
    g = GOLDEN[case]
    dtype = torch.int16 if g.get("dtype") == "int16" else torch.float32
    # int16 goldens are raw bf16 words: run them as bf16 tensors.
    run_dtype = torch.bfloat16 if dtype == torch.int16 else torch.float32
    key = torch.tensor(g["key"], dtype=dtype).view(run_dtype).to(gpu_device)
    value = torch.tensor(g["value"], dtype=dtype).view(run_dtype).to(gpu_device)
    kc = torch.full(g["cache_shape"], g["cache_fill"], dtype=dtype).view(run_dtype).to(gpu_device)
    vc = kc.clone()
    slots = torch.tensor(g["slot_mapping"], dtype=torch.int32, device=gpu_device)
    backend.store(key, value, kc, vc, slots)
    exp_k = np.asarray(g["expected_key_cache"], dtype=np.int16 if dtype == torch.int16 else np.float32)
    exp_v = np.asarray(g["expected_value_cache"], dtype=exp_k.dtype)
    np.testing.assert_array_equal(kc.cpu().view(dtype).numpy(), exp_k)
    np.testing.assert_array_equal(vc.cpu().view(dtype).numpy(), exp_v)
    if "expected_gather" in g:
        table = torch.tensor(g["block_table"], dtype=torch.int32, device=gpu_device)
        got = backend.gather(kc, table, g["sequence_length"]).cpu().view(dtype).numpy()
        np.testing.assert_array_equal(got, np.asarray(g["expected_gather"], dtype=exp_k.dtype))


@pytest.mark.parametrize("case", ["gather", "sdpa_gather"])
def test_gather_goldens_on_gpu(backend, gpu_device, case):
    g = GOLDEN[case]
    cache = torch.tensor(g["cache"], dtype=torch.float32, device=gpu_device)
    table = torch.tensor(g["block_table"], dtype=torch.int32, device=gpu_device)
    got = backend.gather(cache, table, g["sequence_length"]).cpu().numpy()
    np.testing.assert_array_equal(got, np.asarray(g["expected"], dtype=np.float32))


# -------------------------------------------------------------- edge cases

def test_empty_store_and_zero_length_gather(backend, gpu_device):
    kc = torch.zeros(3, 4, 2, 8, dtype=torch.bfloat16, device=gpu_device)
    vc = torch.zeros_like(kc)
    empty = torch.empty(0, 2, 8, dtype=torch.bfloat16, device=gpu_device)
    backend.store(empty, empty, kc, vc, torch.empty(0, dtype=torch.int32, device=gpu_device))
    assert int(kc.count_nonzero()) == 0
    out = backend.gather(kc, torch.tensor([1], dtype=torch.int32, device=gpu_device), 0)
    assert tuple(out.shape) == (0, 2, 8)
    k_out, v_out = backend.gather_varlen(
        kc, vc, torch.full((2, 1), -1, dtype=torch.int32, device=gpu_device),
        torch.zeros(3, dtype=torch.int32, device=gpu_device), 0,
    )
    assert k_out.shape[0] == 0 and v_out.shape[0] == 0


def test_out_of_range_indices_never_touch_memory(backend, gpu_device, monkeypatch):
    """With index validation off (the default on GPU), a slot outside
    [-1, NB*BS) is skipped like -1 and an invalid physical block gathers
    zero rows; with validation on, both raise ValueError as in the
    reference (base.py:104-107, 139-144)."""
    monkeypatch.delenv("NANOVLLM_PAGED_KV_VALIDATE_INDICES", raising=False)
    kc = torch.full((2, 4, 1, 8), 7, dtype=torch.float16, device=gpu_device)
    vc = kc.clone()
    key = torch.ones(3, 1, 8, dtype=torch.float16, device=gpu_device)
    slots = torch.tensor([8, -7, 1], dtype=torch.int32, device=gpu_device)
    backend.store(key, key, kc, vc, slots)
    expected = torch.full((2, 4, 1, 8), 7, dtype=torch.float16)
    expected[0, 1] = 1
    assert torch.equal(kc.cpu(), expected)
    out = backend.gather(kc, torch.tensor([1, 5], dtype=torch.int32, device=gpu_device), 6)
    assert torch.equal(out[:4].cpu(), kc[1].cpu())
    assert int(out[4:].count_nonzero()) == 0
    monkeypatch.setenv("NANOVLLM_PAGED_KV_VALIDATE_INDICES", "1")
    with pytest.raises(ValueError, match="slot"):
        backend.store(key, key, kc, vc, slots)
    with pytest.raises(ValueError, match="physical block"):
        backend.gather(kc, torch.tensor([1, 5], dtype=torch.int32, device=gpu_device), 6)


@pytest.mark.parametrize("dtype,heads,dim,offset", [
    (torch.float16, 1, 1, 0),     # 2-byte rows
    (torch.float16, 3, 5, 1),     # 30-byte rows, odd element offset
    (torch.float32, 3, 5, 1),     # 60-byte rows
    (torch.bfloat16, 2, 12, 2),   # 48-byte rows, 4-byte aligned
    (torch.bfloat16, 8, 128, 4),  # 2 KiB rows, 8-byte aligned
])
def test_misaligned_rows(backend, gpu_device, dtype, heads, dim, offset):
    g = torch.Generator(device=gpu_device).manual_seed(3)
    nb, bs, t = 9, 8, 40
    base = torch.randn(t * heads * dim + offset, device=gpu_device, generator=g).to(dtype)
    key = base[offset:].view(t, heads, dim)
    value = torch.randn(t, heads, dim, device=gpu_device, generator=g).to(dtype)
    slots = torch.randperm(nb * bs, device=gpu_device, generator=g)[:t].to(torch.int32)
    slots[::5] = -1
    kc = torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(dtype)
    vc = torch.randn_like(kc)
    hk, hv = oracle_store(key, value, kc, vc, slots)
    backend.store(key, value, kc, vc, slots)
    np.testing.assert_array_equal(words(kc), hk)
    np.testing.assert_array_equal(words(vc), hv)
    table = torch.randperm(nb, device=gpu_device, generator=g).to(torch.int32)
    out_base = torch.empty(nb * bs * heads * dim + offset, device=gpu_device, dtype=dtype)
    for length in (1, 7, 8, 9, nb * bs):
        got = backend.gather(kc, table, length)
        np.testing.assert_array_equal(words(got), oracle.gather(hk, table.cpu().numpy(), length))
    del out_base


# ------------------------------------------------------------ varlen gather

def _random_tables(rng, lens, nb, bs, share=0):
    width = max(1, int(max((-(-int(n) // bs)) for n in lens)) if len(lens) else 1)
    tables = np.full((len(lens), width), -1, np.int32)
    perm = rng.permutation(nb)
    shared = perm[:share]
    cursor = share
    for i, n in enumerate(lens):
        need = -(-int(n) // bs)
        own = min(need, share) if i % 2 == 0 else 0
        tables[i, :own] = shared[:own]
        tables[i, own:need] = perm[cursor:cursor + need - own]
        cursor += need - own
    return tables


@pytest.mark.parametrize("dtype,heads,dim,bs", [
    (torch.bfloat16, 8, 128, 256),
    (torch.bfloat16, 2, 128, 256),
    (torch.float16, 1, 64, 16),
    (torch.float32, 2, 80, 16),
    (torch.float16, 3, 5, 4),
])
def test_gather_varlen_matches_per_request_gathers(backend, gpu_device, dtype, heads, dim, bs):
    rng = np.random.default_rng(heads * 1000 + dim + bs)
    lens = rng.integers(0, 3 * bs + 5, 37)
    lens[3] = 0
    lens[4] = bs
    nb = int(sum(-(-int(n) // bs) for n in lens)) + 8
    tables = _random_tables(rng, lens, nb, bs, share=2)
    g = torch.Generator(device=gpu_device).manual_seed(1)
    kc = torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(dtype)
    vc = torch.randn(nb, bs, heads, dim, device=gpu_device, generator=g).to(dtype)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    d_tables = torch.from_numpy(tables).to(gpu_device)
    d_cu = torch.from_numpy(cu).to(gpu_device)
    k_out, v_out = backend.gather_varlen(kc, vc, d_tables, d_cu, int(cu[-1]))
    np.testing.assert_array_equal(words(k_out), oracle.gather_varlen(words(kc), tables, lens))
    np.testing.assert_array_equal(words(v_out), oracle.gather_varlen(words(vc), tables, lens))
    plan = backend.build_gather_plan(kc, d_tables, d_cu, int(cu[-1]))
    k2 = torch.empty_like(k_out)
    v2 = torch.empty_like(v_out)
    backend.gather_varlen(kc, vc, d_tables, d_cu, int(cu[-1]), plan=plan, out=(k2, v2))
    assert torch.equal(k2.view(WORD[dtype]), k_out.view(WORD[dtype]))
    assert torch.equal(v2.view(WORD[dtype]), v_out.view(WORD[dtype]))


# ----------------------------------------------------------------- packing

@pytest.mark.parametrize("case", GOLDEN["packing"], ids=lambda c: c["name"])
def test_packing_goldens_on_gpu(gpu_device, case):
    from nanokv.packing import DevicePacker, SequenceBatch

    bs = case["block_size"]
    packer = DevicePacker(gpu_device, bs)
    seqs = case["seqs"]
    tables = [s["block_table"] for s in seqs]
    if case.get("decode"):
        batch = SequenceBatch.from_block_lists([s["num_tokens"] for s in seqs], tables)
        ctx = packer.pack_decode(batch)
        assert ctx.slot_mapping.cpu().tolist() == case["slot_mapping"]
        assert ctx.context_lens.cpu().tolist() == case["context_lens"]
        assert ctx.block_tables.cpu().tolist() == case["block_tables"]
        assert ctx.cu_seqlens_k.cpu().tolist() == case["cu_seqlens_k"]
        return
    batch = SequenceBatch.from_block_lists(
        [s["num_cached"] + s["num_scheduled"] for s in seqs], tables,
        num_prompt_tokens=[s["num_prompt"] for s in seqs],
        num_cached_tokens=[s["num_cached"] for s in seqs],
        num_scheduled_tokens=[s["num_scheduled"] for s in seqs],
    )
    ctx = packer.pack_prefill(batch)
    assert ctx.slot_mapping.cpu().tolist() == case["slot_mapping"]
    assert ctx.cu_seqlens_q.cpu().tolist() == case["cu_seqlens_q"]
    assert ctx.cu_seqlens_k.cpu().tolist() == case["cu_seqlens_k"]
    assert ctx.full_context_lens.cpu().tolist() == case["full_context_lens"]
    assert ctx.query_start_lens.cpu().tolist() == case["query_start_lens"]
    assert (ctx.max_seqlen_q, ctx.max_seqlen_k) == (case["max_seqlen_q"], case["max_seqlen_k"])
    if case["block_tables"] is None:
        assert ctx.block_tables is None
    else:
        assert ctx.block_tables.cpu().tolist() == case["block_tables"]


@pytest.mark.parametrize("num_seqs,bs,seed", [(1, 256, 0), (37, 16, 1), (512, 256, 2), (4096, 16, 3)])
def test_pack_decode_and_prefill_random_batches(gpu_device, num_seqs, bs, seed):
    from nanokv.packing import DevicePacker, SequenceBatch

    rng = np.random.default_rng(seed)
    packer = DevicePacker(gpu_device, bs)
    # decode
    n = rng.integers(1, 40 * bs, num_seqs)
    need = (n + bs - 1) // bs
    perm = rng.permutation(int(need.sum()) + 5)
    offsets = np.concatenate([[0], np.cumsum(need)])
    tables = [perm[offsets[i]:offsets[i + 1]].tolist() for i in range(num_seqs)]
    ctx = packer.pack_decode(SequenceBatch.from_block_lists(n, tables))
    seqs = [oracle.SeqState(int(n[i]), tables[i]) for i in range(num_seqs)]
    exp = oracle.prepare_decode(seqs, bs)
    for key in ("slot_mapping", "context_lens", "block_tables", "cu_seqlens_k"):
        np.testing.assert_array_equal(getattr(ctx, key).cpu().numpy(), exp[key], err_msg=key)
    # prefill: continuing sequences, some warmup (empty tables)
    cached = np.where(rng.random(num_seqs) < 0.5, rng.integers(0, 4, num_seqs) * bs, 0)
    q = rng.integers(1, 3 * bs, num_seqs)
    empty = rng.random(num_seqs) < 0.05
    need = (cached + q + bs - 1) // bs
    need[empty] = 0
    perm = rng.permutation(int(need.sum()) + 3)
    offsets = np.concatenate([[0], np.cumsum(need)])
    tables = [perm[offsets[i]:offsets[i + 1]].tolist() for i in range(num_seqs)]
    batch = SequenceBatch.from_block_lists(
        cached + q, tables, num_prompt_tokens=cached + q + 1, num_cached_tokens=cached,
        num_scheduled_tokens=q,
    )
    ctx = packer.pack_prefill(batch)
    seqs = [oracle.SeqState(int(cached[i] + q[i]), tables[i], int(cached[i] + q[i] + 1),
                            int(cached[i]), int(q[i])) for i in range(num_seqs)]
    exp = oracle.prepare_prefill(seqs, bs)
    for key in ("slot_mapping", "cu_seqlens_q", "cu_seqlens_k", "full_context_lens", "query_start_lens"):
        np.testing.assert_array_equal(getattr(ctx, key).cpu().numpy(), exp[key], err_msg=key)
    assert (ctx.max_seqlen_q, ctx.max_seqlen_k) == (exp["max_seqlen_q"], exp["max_seqlen_k"])
    if exp["block_tables"] is None:
        assert ctx.block_tables is None
    else:
        np.testing.assert_array_equal(ctx.block_tables.cpu().numpy(), exp["block_tables"])


# ------------------------------------------------------ full-size workloads

def _compact(cache: torch.Tensor, blocks: np.ndarray):
    """Host copy of only the referenced blocks of a device cache, with the
    map physical block -> compact index (the oracle needs no more)."""
    blocks = np.unique(blocks[blocks >= 0])
    index = torch.from_numpy(blocks.astype(np.int64)).to(cache.device)
    host = cache.index_select(0, index).cpu().contiguous().view(WORD[cache.dtype]).numpy()
    remap = np.full(cache.shape[0], -1, np.int64)
    remap[blocks] = np.arange(blocks.size)
    return host, remap


def _remap_tables(tables: np.ndarray, remap: np.ndarray) -> np.ndarray:
    out = tables.copy()
    mask = out >= 0
    out[mask] = remap[out[mask]]
    return out.astype(np.int32)


def _remap_slots(slots: np.ndarray, remap: np.ndarray, bs: int) -> np.ndarray:
    out = slots.astype(np.int64).copy()
    mask = out >= 0
    out[mask] = remap[out[mask] // bs] * bs + out[mask] % bs
    return out.astype(np.int32)


def _fill_random(cache: torch.Tensor, seed: int) -> None:
    g = torch.Generator(device=cache.device).manual_seed(seed)
    cache.view(WORD[cache.dtype]).random_(-32768, 32767, generator=g)


@pytest.mark.parametrize("name,overrides", [
    ("decode_store", {}), ("chunked_prefill", {}), ("narrow_rows", {}),
    # the narrow-row batch with the shared blocks filled in the step itself,
    # an order the reference's scheduler never produces: store then gather
    # still equals the oracle on it
    ("narrow_rows", {"schedule": "same_step"}),
])
def test_workload_store_then_gather_full_size(backend, gpu_device, name, overrides):
    from nanokv import workloads
    from nanokv.packing import DevicePacker, SequenceBatch

    wl = workloads.build(name, **overrides)
    print(f"[workload {name} {overrides}] seqs={wl.num_seqs} blocks={wl.num_blocks}", flush=True)
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    kc = torch.empty(shape, dtype=wl.dtype, device=gpu_device)
    vc = torch.empty_like(kc)
    _fill_random(kc, 1)
    _fill_random(vc, 2)
    tables = wl.padded_block_tables()
    used = np.unique(np.concatenate([tables.ravel(), wl.slot_mapping[wl.slot_mapping >= 0] // wl.block_size]))
    hk, remap = _compact(kc, used)
    hv, _ = _compact(vc, used)

    # Slots packed on the device equal the workload's slots.
    offsets, ids = wl.csr()
    packer = DevicePacker(gpu_device, wl.block_size)
    if wl.phase == "decode":
        ctx = packer.pack_decode(SequenceBatch(wl.num_tokens, offsets, ids))
        valid = wl.slot_mapping >= 0
        np.testing.assert_array_equal(ctx.slot_mapping.cpu().numpy()[valid], wl.slot_mapping[valid])
    else:
        ctx = packer.pack_prefill(SequenceBatch(
            wl.num_tokens, offsets, ids, wl.num_prompt, wl.num_cached, wl.num_scheduled))
        np.testing.assert_array_equal(ctx.slot_mapping.cpu().numpy(), wl.slot_mapping)

    slots = torch.from_numpy(wl.slot_mapping).to(gpu_device)
    key, value = wl.key.to(gpu_device), wl.value.to(gpu_device)
    backend.store(key, value, kc, vc, slots)
    c_oracle.store(words(wl.key), words(wl.value), hk, hv,
                   _remap_slots(wl.slot_mapping, remap, wl.block_size), threads=8)
    got_k, _ = _compact(kc, used)
    got_v, _ = _compact(vc, used)
    np.testing.assert_array_equal(got_k, hk)
    np.testing.assert_array_equal(got_v, hv)

    if wl.phase == "decode":
        return
    lens = wl.context_lens
    cu = wl.cu_seqlens_k()
    k_out, v_out = backend.gather_varlen(kc, vc, torch.from_numpy(tables).to(gpu_device),
                                         torch.from_numpy(cu).to(gpu_device), int(cu[-1]))
    ctables = _remap_tables(tables, remap)
    np.testing.assert_array_equal(words(k_out), c_oracle.gather_varlen(hk, ctables, cu, threads=8))
    np.testing.assert_array_equal(words(v_out), c_oracle.gather_varlen(hv, ctables, cu, threads=8))
    del lens


def test_prefix_gather_full_size(backend, gpu_device):
    from nanokv import workloads

    wl = workloads.build("prefix_gather")
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    print(f"[workload prefix_gather] tokens={int(wl.context_lens.sum())}", flush=True)
    kc = torch.empty(shape, dtype=wl.dtype, device=gpu_device)
    vc = torch.empty_like(kc)
    _fill_random(kc, 3)
    _fill_random(vc, 4)
    tables = wl.padded_block_tables()
    hk, remap = _compact(kc, tables.ravel())
    hv, _ = _compact(vc, tables.ravel())
    ctables = _remap_tables(tables, remap)
    cu = wl.cu_seqlens_k()
    d_tables = torch.from_numpy(tables).to(gpu_device)
    k_out, v_out = backend.gather_varlen(kc, vc, d_tables, torch.from_numpy(cu).to(gpu_device), int(cu[-1]))
    np.testing.assert_array_equal(words(k_out), c_oracle.gather_varlen(hk, ctables, cu, threads=8))
    np.testing.assert_array_equal(words(v_out), c_oracle.gather_varlen(hv, ctables, cu, threads=8))
    # The reference-op path: one gather per sequence (attention.py:254-259).
    for i in (0, 1, 7, 30):
        n = int(wl.context_lens[i])
        need = -(-n // wl.block_size)
        got = backend.gather(kc, d_tables[i, :need].contiguous(), n)
        np.testing.assert_array_equal(words(got), oracle.gather(hk, ctables[i], n))


def test_decode_step_full_size_two_layers(backend, gpu_device):
    """The decode-step pipeline at the real per-layer size (256 contexts,
    ~4k blocks): device packing, then per layer store + planned varlen
    gather of K and V, checked against the oracle for every row of two
    layers."""
    from nanokv import workloads
    from nanokv.packing import DevicePacker, SequenceBatch

    wl = workloads.build("decode_step", num_layers=2)
    print(f"[workload decode_step] blocks={wl.num_blocks} tokens={int(wl.num_tokens.sum())}", flush=True)
    shape = (2, wl.num_layers, wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    cache = torch.empty(shape, dtype=wl.dtype, device=gpu_device)
    _fill_random(cache, 5)
    offsets, ids = wl.csr()
    ctx = DevicePacker(gpu_device, wl.block_size).pack_decode(SequenceBatch(wl.num_tokens, offsets, ids))
    np.testing.assert_array_equal(ctx.slot_mapping.cpu().numpy(), wl.slot_mapping)
    tables = wl.padded_block_tables()
    np.testing.assert_array_equal(ctx.block_tables.cpu().numpy(), tables)
    total = ctx.total_context_tokens
    plan = backend.build_gather_plan(cache[0, 0], ctx.block_tables, ctx.cu_seqlens_k, total)
    k_out = torch.empty((total, wl.num_kv_heads, wl.head_dim), dtype=wl.dtype, device=gpu_device)
    v_out = torch.empty_like(k_out)
    cu = wl.cu_seqlens_k()
    for layer in range(wl.num_layers):
        kc, vc = cache[0, layer], cache[1, layer]
        hk, remap = _compact(kc, tables.ravel())
        hv, _ = _compact(vc, tables.ravel())
        key, value = wl.key[layer].to(gpu_device), wl.value[layer].to(gpu_device)
        backend.store(key, value, kc, vc, ctx.slot_mapping)
        backend.gather_varlen(kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total, plan=plan, out=(k_out, v_out))
        c_oracle.store(words(wl.key[layer]), words(wl.value[layer]), hk, hv,
                       _remap_slots(wl.slot_mapping, remap, wl.block_size), threads=8)
        ctables = _remap_tables(tables, remap)
        np.testing.assert_array_equal(words(k_out), c_oracle.gather_varlen(hk, ctables, cu, threads=8))
        np.testing.assert_array_equal(words(v_out), c_oracle.gather_varlen(hv, ctables, cu, threads=8))


def test_store_gather_above_4gib_offsets(backend, gpu_device):
    """Rows past 4 GiB into a cache (8192 blocks of 256 rows of 2 KiB per
    cache, 4 GiB each): the store's, the gather's and the fused
    store+gather's byte offsets need 64 bits there."""
    nb, bs, heads, dim = 8192, 256, 8, 128
    kc = torch.zeros((nb, bs, heads, dim), dtype=torch.bfloat16, device=gpu_device)
    vc = torch.zeros_like(kc)
    top = np.arange(nb - 3, nb, dtype=np.int32)                 # the last three blocks
    rng = np.random.default_rng(4)
    slots = np.concatenate([top[2] * bs + np.arange(bs - 40, bs), top[0] * bs + rng.permutation(bs)[:30]])
    slots = slots.astype(np.int32)
    slots[[3, 17]] = -1
    g = torch.Generator(device=gpu_device).manual_seed(6)
    key = torch.randn((slots.size, heads, dim), device=gpu_device, generator=g).to(torch.bfloat16)
    value = torch.randn_like(key)
    backend.store(key, value, kc, vc, torch.from_numpy(slots).to(gpu_device))
    hk = np.zeros((3, bs, heads, dim), np.int16)
    hv = np.zeros_like(hk)
    local = np.where(slots >= 0, (slots // bs - (nb - 3)) * bs + slots % bs, -1).astype(np.int32)
    oracle.store(words(key), words(value), hk, hv, local)
    np.testing.assert_array_equal(words(kc[nb - 3:]), hk)
    np.testing.assert_array_equal(words(vc[nb - 3:]), hv)
    table = torch.tensor([nb - 1, nb - 3, nb - 2], dtype=torch.int32, device=gpu_device)
    length = 2 * bs + 77
    np.testing.assert_array_equal(words(backend.gather(kc, table, length)),
                                  oracle.gather(hk, np.array([2, 0, 1]), length))
    # the fused op on one request whose new rows are the last 40 of block nb-1
    cu_q = torch.tensor([0, 40], dtype=torch.int32, device=gpu_device)
    cu_k = torch.tensor([0, bs], dtype=torch.int32, device=gpu_device)
    tables = torch.tensor([[nb - 1]], dtype=torch.int32, device=gpu_device)
    new_k = torch.randn((40, heads, dim), device=gpu_device, generator=g).to(torch.bfloat16)
    new_v = torch.randn_like(new_k)
    fused_slots = torch.from_numpy(((nb - 1) * bs + np.arange(bs - 40, bs)).astype(np.int32)).to(gpu_device)
    k_out, v_out = backend.store_gather(new_k, new_v, kc, vc, fused_slots, tables, cu_q, cu_k, bs)
    oracle.store(words(new_k), words(new_v), hk, hv, (2 * bs + np.arange(bs - 40, bs)).astype(np.int32))
    np.testing.assert_array_equal(words(k_out), oracle.gather(hk, np.array([2]), bs))
    np.testing.assert_array_equal(words(v_out), oracle.gather(hv, np.array([2]), bs))
    np.testing.assert_array_equal(words(kc[nb - 3:]), hk)
