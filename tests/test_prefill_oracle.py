"""Pins the prefill-attention oracle (oracle.paged_kv.paged_attention_prefill)
on the CPU:
  * it equals torch's scaled_dot_product_attention in float32 with
    enable_gqa=True and the prefix-causal mask of the reference's SDPA
    prefill (key t visible to query j when t <= Lk - Lq + j;
    nanovllm/layers/attention.py:155-161), on gathered contexts;
  * with Lq == Lk it equals SDPA's own is_causal=True;
  * with one query per request (Lq == 1) it equals the decode oracle;
  * a brute-force loop with math.exp on a tiny case;
  * planted mistakes (top-left instead of bottom-right causal alignment, a
    wrong GQA head mapping) are caught.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_kv as oracle


def bf16_words(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy()


def make_case(seed, q_lens, k_lens, nb=40, bs=4, hkv=2, g=2, d=16):
    gen = torch.Generator().manual_seed(seed)
    b = len(q_lens)
    kc = torch.randn(nb, bs, hkv, d, generator=gen)
    vc = torch.randn(nb, bs, hkv, d, generator=gen)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    q = torch.randn(int(cu_q[-1]), hkv * g, d, generator=gen).to(torch.bfloat16).float()
    width = max(1, max(-(-n // bs) for n in k_lens))
    tables = np.full((b, width), -1, np.int32)
    perm = torch.randperm(nb, generator=gen).numpy()
    cursor = 0
    for i, n in enumerate(k_lens):
        need = -(-n // bs)
        tables[i, :need] = perm[cursor:cursor + need]
        cursor += need
    return q, cu_q, bf16_words(kc), bf16_words(vc), tables, cu_k


def context(cache, table, n):
    return torch.from_numpy(oracle.bf16_words_to_f32(oracle.gather(cache, table, n)))


@pytest.mark.parametrize("hkv,g", [(2, 2), (1, 4), (4, 1)])
def test_oracle_equals_torch_sdpa_prefix_causal(hkv, g):
    q_lens, k_lens = [3, 1, 5, 7, 2], [9, 1, 5, 12, 8]
    q, cu_q, kc, vc, tables, cu_k = make_case(7 + hkv + g, q_lens, k_lens, hkv=hkv, g=g)
    scale = 1.0 / math.sqrt(q.shape[-1])
    got = oracle.paged_attention_prefill(q.numpy(), cu_q, kc, vc, tables, cu_k, scale)
    for i, (lq, lk) in enumerate(zip(q_lens, k_lens)):
        k, v = context(kc, tables[i], lk), context(vc, tables[i], lk)
        query_pos = torch.arange(lq) + (lk - lq)
        mask = torch.arange(lk)[None, :] <= query_pos[:, None]
        expected = F.scaled_dot_product_attention(
            q[cu_q[i]:cu_q[i + 1]].transpose(0, 1).unsqueeze(0),  # [1, Hq, Lq, D]
            k.transpose(0, 1).unsqueeze(0).contiguous(),          # [1, Hkv, Lk, D]
            v.transpose(0, 1).unsqueeze(0).contiguous(),
            attn_mask=mask.unsqueeze(0).unsqueeze(0), scale=scale, enable_gqa=True,
        )[0].transpose(0, 1)
        np.testing.assert_allclose(got[cu_q[i]:cu_q[i + 1]], expected.numpy(), rtol=1e-5, atol=1e-6)


def test_full_prompt_equals_sdpa_is_causal():
    lens = [6, 1, 13]
    q, cu_q, kc, vc, tables, cu_k = make_case(21, lens, lens)
    got = oracle.paged_attention_prefill(q.numpy(), cu_q, kc, vc, tables, cu_k, 0.3)
    for i, n in enumerate(lens):
        k, v = context(kc, tables[i], n), context(vc, tables[i], n)
        expected = F.scaled_dot_product_attention(
            q[cu_q[i]:cu_q[i + 1]].transpose(0, 1).unsqueeze(0),
            k.transpose(0, 1).unsqueeze(0).contiguous(),
            v.transpose(0, 1).unsqueeze(0).contiguous(),
            is_causal=True, scale=0.3, enable_gqa=True,
        )[0].transpose(0, 1)
        np.testing.assert_allclose(got[cu_q[i]:cu_q[i + 1]], expected.numpy(), rtol=1e-5, atol=1e-6)


def test_one_query_per_request_equals_decode_oracle():
    k_lens = [1, 4, 9, 17]
    q, cu_q, kc, vc, tables, cu_k = make_case(5, [1] * 4, k_lens, hkv=2, g=4)
    prefill = oracle.paged_attention_prefill(q.numpy(), cu_q, kc, vc, tables, cu_k, 0.25)
    decode = oracle.paged_attention_decode(q.numpy(), kc, vc, tables, np.array(k_lens), 0.25)
    np.testing.assert_allclose(prefill, decode, rtol=1e-6, atol=1e-7)


def test_brute_force_loop():
    q, cu_q, kc, vc, tables, cu_k = make_case(9, [3], [5], hkv=1, g=2, d=4)
    scale = 0.5
    got = oracle.paged_attention_prefill(q.numpy(), cu_q, kc, vc, tables, cu_k, scale)
    k = oracle.bf16_words_to_f32(oracle.gather(kc, tables[0], 5))
    v = oracle.bf16_words_to_f32(oracle.gather(vc, tables[0], 5))
    for j in range(3):
        last = 5 - 3 + j
        for h in range(2):
            scores = [scale * sum(float(q[j, h, e]) * float(k[t, 0, e]) for e in range(4))
                      for t in range(last + 1)]
            top = max(scores)
            w = [math.exp(s - top) for s in scores]
            for e in range(4):
                expected = sum(w[t] * float(v[t, 0, e]) for t in range(last + 1)) / sum(w)
                assert abs(got[j, h, e] - expected) < 1e-5


def test_planted_mistakes_are_caught():
    q, cu_q, kc, vc, tables, cu_k = make_case(11, [4], [10], hkv=2, g=2)
    scale = 0.3
    good = oracle.paged_attention_prefill(q.numpy(), cu_q, kc, vc, tables, cu_k, scale)
    k = oracle.bf16_words_to_f32(oracle.gather(kc, tables[0], 10))
    v = oracle.bf16_words_to_f32(oracle.gather(vc, tables[0], 10))
    qn = q.numpy()

    def attend(j, h, kv, last):
        s = (k[: last + 1, kv] @ qn[j, h]) * scale
        p = np.exp(s - s.max())
        return (p / p.sum()) @ v[: last + 1, kv]

    top_left = np.stack([[attend(j, h, h // 2, j) for h in range(4)] for j in range(4)])
    assert not np.allclose(top_left, good, atol=1e-3)
    wrong_heads = np.stack([[attend(j, h, h % 2, 10 - 4 + j) for h in range(4)] for j in range(4)])
    assert not np.allclose(wrong_heads, good, atol=1e-3)
    right = np.stack([[attend(j, h, h // 2, 10 - 4 + j) for h in range(4)] for j in range(4)])
    np.testing.assert_allclose(right, good, rtol=1e-5, atol=1e-6)


def test_float16_words_and_oracle_equal_torch():
    """The fp16 path: the word conversion equals torch's float16 -> float32
    for every finite and special pattern, and the oracle on float16 caches
    equals SDPA with the prefix-causal mask on the same values, taken from
    torch directly."""
    words = np.arange(-32768, 32768, dtype=np.int64).astype(np.int16)
    expect = torch.from_numpy(words).view(torch.float16).float().numpy()
    got = oracle.words_to_f32(words, "float16")
    both_nan = np.isnan(got) & np.isnan(expect)
    np.testing.assert_array_equal(got[~both_nan], expect[~both_nan])

    q_lens, k_lens = [3, 5, 2], [9, 5, 8]
    gen = torch.Generator().manual_seed(5)
    nb, bs, hkv, g, d = 12, 4, 2, 2, 16
    kc = torch.randn(nb, bs, hkv, d, generator=gen).to(torch.float16)
    vc = torch.randn(nb, bs, hkv, d, generator=gen).to(torch.float16)
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    q = torch.randn(int(cu_q[-1]), hkv * g, d, generator=gen).to(torch.float16).float()
    tables = np.array([[0, 1, 2], [3, 4, -1], [5, 6, -1]], np.int32)
    scale = 1.0 / math.sqrt(d)
    out = oracle.paged_attention_prefill(q.numpy(), cu_q, kc.view(torch.int16).numpy(),
                                         vc.view(torch.int16).numpy(), tables, cu_k, scale,
                                         dtype="float16")
    for i, (lq, lk) in enumerate(zip(q_lens, k_lens)):
        rows = [int(tables[i][t // bs]) * bs + t % bs for t in range(lk)]
        k = kc.flatten(0, 1)[rows].float()
        v = vc.flatten(0, 1)[rows].float()
        mask = torch.arange(lk)[None, :] <= (torch.arange(lq) + (lk - lq))[:, None]
        expected = F.scaled_dot_product_attention(
            q[cu_q[i]:cu_q[i + 1]].transpose(0, 1).unsqueeze(0),
            k.transpose(0, 1).unsqueeze(0).contiguous(), v.transpose(0, 1).unsqueeze(0).contiguous(),
            attn_mask=mask.unsqueeze(0).unsqueeze(0), scale=scale, enable_gqa=True,
        )[0].transpose(0, 1)
        np.testing.assert_allclose(out[cu_q[i]:cu_q[i + 1]], expected.numpy(), rtol=1e-5, atol=1e-6)
