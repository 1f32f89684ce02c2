"""Writes tests/golden/paged_kv_golden.json: known-answer vectors for the
paged-KV store / gather / packing path.

Every vector re-enters a known answer that the reference's own tests state
(file:line given per case) or a hand-derived one, and every expected value
is built here by explicit placement (block = slot // BS, offset = slot % BS;
output row t = cache[table[t // BS], t % BS]) or typed in by hand.  This
script imports neither the oracle nor the reference, so the fixtures are an
independent statement of the answers.
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent / "paged_kv_golden.json"


def _place(cache: np.ndarray, slot: int, row: np.ndarray) -> None:
    block_size = cache.shape[1]
    cache[slot // block_size, slot % block_size] = row


def store_known_answer():
    """tests/test_paged_kv_backends.py:17-23, 128-137: arange keys 3x2x4,
    V = K + 100, caches (3,4,2,4) filled -1, slots [0, 5, -1]: flat rows 0
    and 5 receive tokens 0 and 1, token 2 is skipped."""
    key = np.arange(24, dtype=np.float32).reshape(3, 2, 4)
    value = key + 100
    expected_k = np.full((3, 4, 2, 4), -1, dtype=np.float32)
    expected_v = np.full((3, 4, 2, 4), -1, dtype=np.float32)
    expected_k[0, 0] = key[0]
    expected_k[1, 1] = key[1]  # flat row 5 = block 1, offset 1
    expected_v[0, 0] = value[0]
    expected_v[1, 1] = value[1]
    return {
        "key": key.tolist(), "value": value.tolist(), "cache_shape": [3, 4, 2, 4],
        "cache_fill": -1.0, "slot_mapping": [0, 5, -1],
        "expected_key_cache": expected_k.tolist(), "expected_value_cache": expected_v.tolist(),
        "source": "tests/test_paged_kv_backends.py:17-23,128-137",
    }


def gather_known_answer():
    """tests/test_paged_kv_backends.py:139-147: arange cache (3,4,2,4),
    table [2, 0], L = 6 -> cat(cache[2], cache[0])[:6]."""
    cache = np.arange(96, dtype=np.float32).reshape(3, 4, 2, 4)
    expected = np.concatenate([cache[2], cache[0]], axis=0)[:6]
    return {
        "cache": cache.tolist(), "block_table": [2, 0], "sequence_length": 6,
        "expected": expected.tolist(), "source": "tests/test_paged_kv_backends.py:139-147",
    }


def sdpa_gather_known_answer():
    """tests/test_sdpa_attention.py:31-39: arange cache (3,4,1,2), table
    [2, 0], L = 6."""
    cache = np.arange(24, dtype=np.float32).reshape(3, 4, 1, 2)
    expected = np.concatenate([cache[2], cache[0]], axis=0)[:6]
    return {
        "cache": cache.tolist(), "block_table": [2, 0], "sequence_length": 6,
        "expected": expected.tolist(), "source": "tests/test_sdpa_attention.py:31-39",
    }


def slot_matrix_known_answer():
    """The slot / table pattern of tests/test_paged_kv_cuda.py:22-46
    (slots [0,17,-1,4,31,8,23,2,15], caches (4,8,H,D) filled -3, table
    [3,1,0], L = 19) with deterministic rows: key row t holds 1000*t + j,
    value row t holds -(1000*t + j)."""
    heads, dim = 2, 4
    slots = [0, 17, -1, 4, 31, 8, 23, 2, 15]
    key = (1000 * np.arange(9)[:, None] + np.arange(heads * dim)[None, :]).astype(np.float32)
    key = key.reshape(9, heads, dim)
    value = -key
    cache_k = np.full((4, 8, heads, dim), -3, dtype=np.float32)
    cache_v = np.full((4, 8, heads, dim), -3, dtype=np.float32)
    for t, slot in enumerate(slots):
        if slot >= 0:
            _place(cache_k, slot, key[t])
            _place(cache_v, slot, value[t])
    table = [3, 1, 0]
    gathered = np.stack([cache_k[table[t // 8], t % 8] for t in range(19)])
    return {
        "key": key.tolist(), "value": value.tolist(), "cache_shape": [4, 8, heads, dim],
        "cache_fill": -3.0, "slot_mapping": slots, "expected_key_cache": cache_k.tolist(),
        "expected_value_cache": cache_v.tolist(), "block_table": table, "sequence_length": 19,
        "expected_gather": gathered.tolist(), "source": "tests/test_paged_kv_cuda.py:22-46",
    }


def native_allocation_known_answer():
    """tests/test_paged_kv_cuda.py:155-185: caches (5,8,2,128) filled -5,
    slots [0,9,17,-1,31,2,7,20,39,12], table [4,1,3], L = 19, with
    deterministic rows (key row t = 100*t + j mod 2^15 as int16 words)."""
    heads, dim = 2, 128
    slots = [0, 9, 17, -1, 31, 2, 7, 20, 39, 12]
    words = (100 * np.arange(10)[:, None] + np.arange(heads * dim)[None, :]) % 32768
    key = words.astype(np.int16).reshape(10, heads, dim)
    value = (-key).astype(np.int16)
    cache_k = np.full((5, 8, heads, dim), -5, dtype=np.int16)
    cache_v = np.full((5, 8, heads, dim), -5, dtype=np.int16)
    for t, slot in enumerate(slots):
        if slot >= 0:
            _place(cache_k, slot, key[t])
            _place(cache_v, slot, value[t])
    table = [4, 1, 3]
    gathered = np.stack([cache_k[table[t // 8], t % 8] for t in range(19)])
    return {
        "key": key.tolist(), "value": value.tolist(), "cache_shape": [5, 8, heads, dim],
        "cache_fill": -5, "slot_mapping": slots, "expected_key_cache": cache_k.tolist(),
        "expected_value_cache": cache_v.tolist(), "block_table": table, "sequence_length": 19,
        "expected_gather": gathered.tolist(), "dtype": "int16",
        "source": "tests/test_paged_kv_cuda.py:155-185",
    }


def decode_replay_known_answer():
    """tests/test_paged_kv_cuda.py:245-273: 64 decode steps, step s stores
    key = s, value = -s at slot s % 16 of a (1,16,1,64) cache: the last 16
    writes win, so key_cache[0, :, 0, 0] = 48..63."""
    return {
        "steps": 64, "cache_shape": [1, 16, 1, 64], "cache_fill": -1.0,
        "expected_key_column": list(range(48, 64)),
        "expected_value_column": [-v for v in range(48, 64)],
        "source": "tests/test_paged_kv_cuda.py:245-273",
    }


def packing_known_answers():
    """Hand-derived packer answers (model_runner.py:757-820, 892-938)."""
    return [
        {
            "name": "prefill_continuation_two_blocks",
            "block_size": 4,
            "seqs": [{"num_cached": 3, "num_scheduled": 4, "num_prompt": 7, "block_table": [7, 2]}],
            # positions 3..6: p=3 -> 7*4+3 = 31; p=4..6 -> 2*4+0..2 = 8, 9, 10
            "slot_mapping": [31, 8, 9, 10], "cu_seqlens_q": [0, 4], "cu_seqlens_k": [0, 7],
            "max_seqlen_q": 4, "max_seqlen_k": 7, "block_tables": [[7, 2]],
            "full_context_lens": [7], "query_start_lens": [3],
        },
        {
            "name": "prefill_three_blocks_and_fresh_sequence",
            "block_size": 4,
            "seqs": [
                {"num_cached": 2, "num_scheduled": 9, "num_prompt": 11, "block_table": [1, 2, 3]},
                {"num_cached": 0, "num_scheduled": 3, "num_prompt": 3, "block_table": [5]},
            ],
            # seq 0: p=2,3 -> 6,7; p=4..7 -> 8..11; p=8..10 -> 12..14
            # seq 1: p=0..2 -> 20, 21, 22
            "slot_mapping": [6, 7, 8, 9, 10, 11, 12, 13, 14, 20, 21, 22],
            "cu_seqlens_q": [0, 9, 12], "cu_seqlens_k": [0, 11, 14],
            "max_seqlen_q": 9, "max_seqlen_k": 11, "block_tables": [[1, 2, 3], [5, -1, -1]],
            "full_context_lens": [11, 3], "query_start_lens": [2, 0],
        },
        {
            "name": "prefill_warmup_sequence_emits_no_slots",
            "block_size": 4,
            "seqs": [
                {"num_cached": 0, "num_scheduled": 3, "num_prompt": 3, "block_table": []},
                {"num_cached": 0, "num_scheduled": 2, "num_prompt": 2, "block_table": [4]},
            ],
            "slot_mapping": [16, 17], "cu_seqlens_q": [0, 3, 5], "cu_seqlens_k": [0, 3, 5],
            "max_seqlen_q": 3, "max_seqlen_k": 3, "block_tables": None,
            "full_context_lens": [3, 2], "query_start_lens": [0, 0],
        },
        {
            "name": "decode_last_token_slots",
            "block_size": 4,
            "decode": True,
            "seqs": [
                # 5 tokens, 2 blocks, 1 token in the last block -> 9*4 + 0
                {"num_tokens": 5, "block_table": [3, 9]},
                # 8 tokens, last block full -> 6*4 + 3
                {"num_tokens": 8, "block_table": [1, 6]},
                # 1 token -> 5*4 + 0
                {"num_tokens": 1, "block_table": [5]},
            ],
            "slot_mapping": [36, 27, 20], "context_lens": [5, 8, 1],
            "block_tables": [[3, 9], [1, 6], [5, -1]], "cu_seqlens_k": [0, 5, 13, 14],
        },
    ]


def benchmark_known_answers():
    """tests/test_bench_paged_kv.py:58-81 (effective_bytes) and :83-89
    (linear percentiles of [1, 2, 3, 4])."""
    return {
        "effective_bytes": [
            {"operation": "store", "tokens": 8, "heads": 2, "dim": 128, "element_size": 2,
             "expected": 8 * 2 * 128 * 2 * 4},
            {"operation": "gather", "tokens": 9, "heads": 1, "dim": 80, "element_size": 4,
             "expected": 9 * 1 * 80 * 4 * 2},
        ],
        "percentiles": {"values": [1.0, 2.0, 3.0, 4.0], "p50": 2.5, "p95": 3.85, "p99": 3.97},
        "source": "tests/test_bench_paged_kv.py:58-89",
    }


def main() -> None:
    payload = {
        "store": store_known_answer(),
        "gather": gather_known_answer(),
        "sdpa_gather": sdpa_gather_known_answer(),
        "slot_matrix": slot_matrix_known_answer(),
        "native_allocation": native_allocation_known_answer(),
        "decode_replay": decode_replay_known_answer(),
        "packing": packing_known_answers(),
        "benchmark": benchmark_known_answers(),
    }
    OUT.write_text(json.dumps(payload, separators=(",", ":")) + "\n")
    print(OUT, OUT.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
