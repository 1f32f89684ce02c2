"""CPU restatement of the reference's paged-KV hot path (numpy and plain
Python).

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, to
check results.  It works on raw element words (any numpy dtype of the right
width; bf16 tensors are passed as int16 views), so every comparison against
it is bit-exact.

Each function cites the reference code it restates.  How each one is pinned
(golden vectors re-entered from the reference's tests, torch's own
index_copy_/index_select on CPU, brute force on tiny inputs, closed-form
invariants) is listed in tests/test_oracle.py.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np


# ---------------------------------------------------------------- store/gather

def store(key, value, key_cache, value_cache, slot_mapping) -> None:
    """nanovllm/layers/paged_kv/pytorch_backend.py:26-38:
    valid = slot >= 0; cache.flatten(0, 1).index_copy_(0, slot[valid], x[valid])
    for K and V.  Arrays: key/value [T, H, D], caches [NB, BS, H, D]
    (modified in place, must be C-contiguous), slot_mapping [T] int32."""
    slots = np.asarray(slot_mapping).astype(np.int64)
    valid = slots >= 0
    kc = key_cache.reshape(-1, *key_cache.shape[2:])
    vc = value_cache.reshape(-1, *value_cache.shape[2:])
    assert np.shares_memory(kc, key_cache) and np.shares_memory(vc, value_cache)
    kc[slots[valid]] = np.asarray(key)[valid]
    vc[slots[valid]] = np.asarray(value)[valid]


def gather(cache, block_table, sequence_length: int):
    """pytorch_backend.py:40-50: cache.index_select(0, table[:ceil(L/BS)])
    .flatten(0, 1)[:L]; [0, H, D] when L == 0."""
    num_blocks, block_size = cache.shape[:2]
    required = -(-sequence_length // block_size)
    if required == 0:
        return np.empty((0, *cache.shape[2:]), dtype=cache.dtype)
    ids = np.asarray(block_table[:required]).astype(np.int64)
    if ids.min() < 0 or ids.max() >= num_blocks:
        raise IndexError("block id out of range")
    return cache[ids].reshape(-1, *cache.shape[2:])[:sequence_length]


def gather_varlen(cache, block_tables, context_lens):
    """Concatenation over requests i of gather(cache, block_tables[i],
    context_lens[i]): the per-request loop of SDPAAttention
    (nanovllm/layers/attention.py:250-259 prefill, 284-292 decode)."""
    parts = [gather(cache, block_tables[i], int(n)) for i, n in enumerate(context_lens)]
    if not parts:
        return np.empty((0, *cache.shape[2:]), dtype=cache.dtype)
    return np.concatenate(parts, axis=0)


def bf16_words_to_f32(words) -> np.ndarray:
    """bf16 bit patterns (int16/uint16 words) -> float32 values (exact)."""
    w = np.asarray(words).astype(np.uint16).astype(np.uint32)
    return (w << 16).view(np.float32)


def words_to_f32(words, dtype: str = "bfloat16") -> np.ndarray:
    """16-bit words of a bfloat16 or float16 tensor -> float32 values (both
    exact: every bf16 and fp16 value is a float32)."""
    if dtype == "bfloat16":
        return bf16_words_to_f32(words)
    if dtype == "float16":
        return np.asarray(words).astype(np.uint16).view(np.float16).astype(np.float32)
    raise ValueError(f"unsupported element type {dtype}")


def paged_attention_decode(q, key_cache, value_cache, block_tables, context_lens, scale: float,
                           dtype: str = "bfloat16"):
    """SDPAAttention's decode branch in float32 (nanovllm/layers/attention.py:
    284-300): per request, gather K and V of its context (the pytorch
    backend's gather, pytorch_backend.py:40-50), then
    softmax(scale * q K^T) V with grouped-query heads: query head h reads kv
    head h // (Hq / Hkv), as scaled_dot_product_attention(enable_gqa=True)
    does (attention.py:194-203).  q [B, Hq, D] float32; caches hold the
    16-bit words of a ``dtype`` tensor ([NB, BS, Hkv, D] int16); an empty
    context yields zeros."""
    q = np.asarray(q, dtype=np.float32)
    b, hq, d = q.shape
    hkv = key_cache.shape[2]
    group = hq // hkv
    out = np.zeros((b, hq, d), dtype=np.float32)
    for i, length in enumerate(np.asarray(context_lens).tolist()):
        if length == 0:
            continue
        k = words_to_f32(gather(key_cache, block_tables[i], int(length)), dtype)
        v = words_to_f32(gather(value_cache, block_tables[i], int(length)), dtype)
        for h in range(hq):
            kv = h // group
            scores = (k[:, kv, :] @ q[i, h]) * np.float32(scale)
            scores = scores - scores.max()
            p = np.exp(scores)
            p /= p.sum()
            out[i, h] = p @ v[:, kv, :]
    return out


def paged_attention_prefill(q, cu_seqlens_q, key_cache, value_cache, block_tables, cu_seqlens_k,
                            scale: float, dtype: str = "bfloat16"):
    """Prefill attention over the paged cache in float32, as the reference's
    prefill computes it when block tables are present: the Flash path reads
    the cache through block_table (nanovllm/layers/attention.py:95-116,
    flash_attn_varlen_func(..., causal=True, block_table=...)); the SDPA path
    gathers each request's keys (:242-251) and applies the prefix-causal
    mask (:155-161, :252-282).  Request i has query rows
    [cu_seqlens_q[i], cu_seqlens_q[i+1]) (Lq of them) and context rows
    [0, Lk), Lk = cu_seqlens_k[i+1] - cu_seqlens_k[i] >= Lq; its query j sits
    at position Lk - Lq + j and attends keys [0, Lk - Lq + j].  Query head h
    reads kv head h // (Hq / Hkv).  q [Tq, Hq, D] float32, caches the 16-bit
    words of a ``dtype`` tensor [NB, BS, Hkv, D]; returns [Tq, Hq, D] float32."""
    q = np.asarray(q, dtype=np.float32)
    tq, hq, d = q.shape
    hkv = key_cache.shape[2]
    group = hq // hkv
    cu_q = np.asarray(cu_seqlens_q).astype(np.int64)
    cu_k = np.asarray(cu_seqlens_k).astype(np.int64)
    out = np.zeros((tq, hq, d), dtype=np.float32)
    for i in range(len(cu_q) - 1):
        q0, lq = int(cu_q[i]), int(cu_q[i + 1] - cu_q[i])
        lk = int(cu_k[i + 1] - cu_k[i])
        if lq == 0:
            continue
        if lk < lq:
            raise ValueError("every request needs at least as many keys as queries")
        k = words_to_f32(gather(key_cache, block_tables[i], lk), dtype)
        v = words_to_f32(gather(value_cache, block_tables[i], lk), dtype)
        visible = np.arange(lk)[None, :] <= (lk - lq + np.arange(lq))[:, None]  # [Lq, Lk]
        for h in range(hq):
            kv = h // group
            scores = (q[q0:q0 + lq, h, :] @ k[:, kv, :].T) * np.float32(scale)
            scores = np.where(visible, scores, -np.inf)
            scores = scores - scores.max(axis=1, keepdims=True)
            p = np.exp(scores)
            p /= p.sum(axis=1, keepdims=True)
            out[q0:q0 + lq, h, :] = p @ v[:, kv, :]
    return out


# --------------------------------------------------------------------- packing

@dataclass
class SeqState:
    """The Sequence fields the packers read (nanovllm/engine/sequence.py:
    98-119, 176-183)."""

    num_tokens: int
    block_table: list[int]
    num_prompt_tokens: int = 0
    num_cached_tokens: int = 0
    num_scheduled_tokens: int = 0

    def num_blocks(self, block_size: int) -> int:
        return (self.num_tokens + block_size - 1) // block_size

    def last_block_num_tokens(self, block_size: int) -> int:
        return self.num_tokens - (self.num_blocks(block_size) - 1) * block_size


def prepare_block_tables(seqs: Sequence[SeqState], width: int | None = None):
    """model_runner.py:696-707: pad every block_table with -1 to the batch
    maximum (or to ``width``), int32 [B, width]."""
    longest = max((len(s.block_table) for s in seqs), default=0)
    width = longest if width is None else width
    assert width >= longest
    table = np.full((len(seqs), width), -1, dtype=np.int32)
    for i, s in enumerate(seqs):
        table[i, : len(s.block_table)] = s.block_table
    return table


def prepare_decode(seqs: Sequence[SeqState], block_size: int, width: int | None = None):
    """model_runner.py:892-938 (metadata part): per sequence
    context_len = len(seq), slot = block_table[-1]*BS + last_block_num_tokens - 1;
    block_tables padded with -1.  Also the exclusive prefix of context_lens
    (cu_seqlens_k) that a varlen gather of the contexts needs."""
    slots = [s.block_table[-1] * block_size + s.last_block_num_tokens(block_size) - 1 for s in seqs]
    context_lens = [s.num_tokens for s in seqs]
    return {
        "slot_mapping": np.array(slots, dtype=np.int32),
        "context_lens": np.array(context_lens, dtype=np.int32),
        "block_tables": prepare_block_tables(seqs, width),
        "cu_seqlens_k": np.concatenate([[0], np.cumsum(context_lens)]).astype(np.int32),
    }


def prepare_prefill(seqs: Sequence[SeqState], block_size: int, width: int | None = None):
    """model_runner.py:757-820, 856-882 (metadata part), following the
    reference's per-block loop literally: start = num_cached, q =
    num_scheduled, end = start + q; sequences with an empty block_table emit
    no slots (warmup); block_tables only when cu_seqlens_k[-1] >
    cu_seqlens_q[-1]."""
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    slots: list[int] = []
    full_context_lens, query_start_lens = [], []
    for s in seqs:
        start = s.num_cached_tokens
        q = s.num_scheduled_tokens
        end = start + q
        full_context_lens.append(s.num_prompt_tokens)
        query_start_lens.append(start)
        cu_q.append(cu_q[-1] + q)
        cu_k.append(cu_k[-1] + end)
        max_q = max(q, max_q)
        max_k = max(end, max_k)
        if not s.block_table:
            continue
        start_block = start // block_size
        end_block = (end + block_size - 1) // block_size
        for i in range(start_block, end_block):
            slot_start = s.block_table[i] * block_size
            if i == start_block:
                slot_start += start % block_size
            if i != end_block - 1:
                slot_end = s.block_table[i] * block_size + block_size
            else:
                slot_end = s.block_table[i] * block_size + end - i * block_size
            slots.extend(range(slot_start, slot_end))
    tables = prepare_block_tables(seqs, width) if cu_k[-1] > cu_q[-1] else None
    return {
        "cu_seqlens_q": np.array(cu_q, dtype=np.int32),
        "cu_seqlens_k": np.array(cu_k, dtype=np.int32),
        "max_seqlen_q": max_q,
        "max_seqlen_k": max_k,
        "slot_mapping": np.array(slots, dtype=np.int32),
        "block_tables": tables,
        "full_context_lens": np.array(full_context_lens, dtype=np.int32),
        "query_start_lens": np.array(query_start_lens, dtype=np.int32),
    }


def graph_replay_fill(graph_buffers: dict, slot_mapping, context_lens, block_tables) -> None:
    """model_runner.py:993-1011: the decode graph's fixed buffers are filled
    as slot_mapping[:] = -1 then [:bs] = slots; context_lens[:] = 0 then
    [:bs] = lens; block_tables[:bs, :w] = tables (columns >= w and rows >=
    bs keep their previous contents)."""
    bs = len(slot_mapping)
    graph_buffers["slot_mapping"][:] = -1
    graph_buffers["slot_mapping"][:bs] = slot_mapping
    graph_buffers["context_lens"][:] = 0
    graph_buffers["context_lens"][:bs] = context_lens
    w = block_tables.shape[1]
    graph_buffers["block_tables"][:bs, :w] = block_tables


def csr(seqs: Sequence[SeqState]):
    """Block lists in the CSR form the device packer takes:
    offsets [B+1] int32, ids [sum of lengths] int32."""
    lengths = [len(s.block_table) for s in seqs]
    offsets = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    ids = np.array([b for s in seqs for b in s.block_table], dtype=np.int32)
    return offsets, ids


# -------------------------------------------------------------- measurement

def effective_bytes(operation: str, num_tokens: int, num_kv_heads: int, head_dim: int,
                    element_size: int) -> int:
    """nanovllm/benchmark/paged_kv.py:196-199: payload x 4 for store (K and V,
    read + write, skipped tokens included), x 2 for gather."""
    payload = num_tokens * num_kv_heads * head_dim * element_size
    return payload * (4 if operation == "store" else 2)


def linear_percentile(values: Sequence[float], quantile: float) -> float:
    """nanovllm/benchmark/metrics.py:82-92."""
    if not values:
        raise ValueError("percentile requires at least one value")
    if not 0.0 <= quantile <= 1.0:
        raise ValueError("quantile must be between zero and one")
    ordered = sorted(values)
    position = (len(ordered) - 1) * quantile
    lower = int(position)
    upper = min(lower + 1, len(ordered) - 1)
    return ordered[lower] + (ordered[upper] - ordered[lower]) * (position - lower)


# ------------------------------------------------------------- brute force

def store_bruteforce(key, value, key_cache, value_cache, slot_mapping) -> None:
    """Row-by-row loop, for tiny inputs: the second, independent statement
    of the store used to pin :func:`store`."""
    block_size = key_cache.shape[1]
    for t, slot in enumerate(np.asarray(slot_mapping).tolist()):
        if slot < 0:
            continue
        block, offset = divmod(slot, block_size)
        key_cache[block, offset] = key[t]
        value_cache[block, offset] = value[t]


def gather_bruteforce(cache, block_table, sequence_length: int):
    """Token-by-token loop: out[t] = cache[table[t // BS], t % BS]."""
    block_size = cache.shape[1]
    out = np.empty((sequence_length, *cache.shape[2:]), dtype=cache.dtype)
    for t in range(sequence_length):
        out[t] = cache[int(block_table[t // block_size]), t % block_size]
    return out


__all__ = [
    "SeqState",
    "bf16_words_to_f32",
    "paged_attention_decode",
    "csr",
    "effective_bytes",
    "gather",
    "gather_bruteforce",
    "gather_varlen",
    "graph_replay_fill",
    "linear_percentile",
    "prepare_block_tables",
    "prepare_decode",
    "prepare_prefill",
    "store",
    "store_bruteforce",
]
