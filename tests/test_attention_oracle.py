"""Pins the decode-attention oracle (oracle.paged_kv.paged_attention_decode)
on the CPU:
  * it equals torch's own scaled_dot_product_attention in float32 with
    enable_gqa=True, called the way SDPAAttention._sdpa calls it
    (nanovllm/layers/attention.py:180-204), on gathered contexts;
  * closed forms: a 1-token context returns that V row; identical keys (or
    q = 0) give uniform weights, i.e. the mean of V; one dominant key
    returns (almost exactly) its V row; an empty context returns zeros;
  * a brute-force loop with math.exp on a tiny case;
  * a planted mistake (kv head h % Hkv instead of h // G) is caught.
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


def make_case(seed, nb=12, bs=4, hkv=2, g=4, d=16, lens=(1, 3, 4, 5, 11, 0)):
    gen = torch.Generator().manual_seed(seed)
    b = len(lens)
    kc = torch.randn(nb, bs, hkv, d, generator=gen)
    vc = torch.randn(nb, bs, hkv, d, generator=gen)
    q = torch.randn(b, hkv * g, d, generator=gen).to(torch.bfloat16).float()
    width = max(1, max((-(-n // bs)) for n in lens))
    tables = np.full((b, width), -1, np.int32)
    perm = torch.randperm(nb, generator=gen).numpy()
    cursor = 0
    for i, n in enumerate(lens):
        need = -(-n // bs)
        tables[i, :need] = perm[cursor:cursor + need]
        cursor += need
    return q, bf16_words(kc), bf16_words(vc), tables, np.array(lens)


@pytest.mark.parametrize("hkv,g", [(2, 4), (1, 2), (4, 1), (2, 1)])
def test_oracle_equals_torch_sdpa_with_gqa(hkv, g):
    q, kc, vc, tables, lens = make_case(3 + hkv + g, hkv=hkv, g=g)
    scale = 1.0 / math.sqrt(q.shape[-1])
    got = oracle.paged_attention_decode(q.numpy(), kc, vc, tables, lens, scale)
    for i, n in enumerate(lens):
        if n == 0:
            assert np.all(got[i] == 0)
            continue
        k = torch.from_numpy(oracle.bf16_words_to_f32(oracle.gather(kc, tables[i], int(n))))
        v = torch.from_numpy(oracle.bf16_words_to_f32(oracle.gather(vc, tables[i], int(n))))
        expected = F.scaled_dot_product_attention(
            q[i:i + 1].transpose(0, 1).unsqueeze(0),      # [1, Hq, 1, D]
            k.transpose(0, 1).unsqueeze(0).contiguous(),  # [1, Hkv, L, D]
            v.transpose(0, 1).unsqueeze(0).contiguous(),
            scale=scale, is_causal=False, enable_gqa=True,
        ).transpose(1, 2).reshape(-1, q.shape[1], q.shape[2])[0]
        np.testing.assert_allclose(got[i], expected.numpy(), rtol=1e-5, atol=1e-6)


def test_closed_forms():
    q, kc, vc, tables, lens = make_case(5, lens=(1, 7))
    scale = 0.25
    out = oracle.paged_attention_decode(q.numpy(), kc, vc, tables, lens, scale)
    v0 = oracle.bf16_words_to_f32(oracle.gather(vc, tables[0], 1))[0]
    for h in range(q.shape[1]):
        np.testing.assert_allclose(out[0, h], v0[h // 4], rtol=0, atol=0)
    # identical keys -> uniform weights -> mean of V
    kc_same = kc.copy()
    kc_same[:] = kc[0, 0]
    out = oracle.paged_attention_decode(q.numpy(), kc_same, vc, tables, lens, scale)
    v1 = oracle.bf16_words_to_f32(oracle.gather(vc, tables[1], 7))
    for h in range(q.shape[1]):
        np.testing.assert_allclose(out[1, h], v1[:, h // 4].mean(axis=0), rtol=1e-5, atol=1e-6)
    # q = 0 -> uniform as well
    out = oracle.paged_attention_decode(np.zeros_like(q.numpy()), kc, vc, tables, lens, scale)
    np.testing.assert_allclose(out[1, 0], v1[:, 0].mean(axis=0), rtol=1e-5, atol=1e-6)
    # one dominant key -> its V row
    k1 = oracle.bf16_words_to_f32(oracle.gather(kc, tables[1], 7))
    qd = np.zeros_like(q.numpy())
    qd[1, 0] = 50.0 * k1[3, 0] / np.linalg.norm(k1[3, 0])
    out = oracle.paged_attention_decode(qd, kc, vc, tables, lens, 1.0)
    weights = np.exp((k1[:, 0] @ qd[1, 0]) - (k1[:, 0] @ qd[1, 0]).max())
    if weights[3] / weights.sum() > 0.999:
        np.testing.assert_allclose(out[1, 0], v1[3, 0], rtol=1e-2, atol=1e-2)


def test_brute_force_loop():
    q, kc, vc, tables, lens = make_case(9, hkv=1, g=2, d=4, lens=(6,))
    scale = 0.5
    got = oracle.paged_attention_decode(q.numpy(), kc, vc, tables, lens, scale)
    k = oracle.bf16_words_to_f32(oracle.gather(kc, tables[0], 6))
    v = oracle.bf16_words_to_f32(oracle.gather(vc, tables[0], 6))
    for h in range(2):
        scores = [scale * sum(float(q[0, h, j]) * float(k[t, 0, j]) for j in range(4)) for t in range(6)]
        top = max(scores)
        w = [math.exp(s - top) for s in scores]
        total = sum(w)
        for j in range(4):
            expected = sum(w[t] * float(v[t, 0, j]) for t in range(6)) / total
            assert abs(got[0, h, j] - expected) < 1e-5


def test_planted_head_mapping_mistake_is_caught():
    q, kc, vc, tables, lens = make_case(11, hkv=2, g=2, lens=(5,))
    scale = 0.3
    good = oracle.paged_attention_decode(q.numpy(), kc, vc, tables, lens, scale)
    # wrong GQA mapping: kv head h % Hkv instead of h // G
    k = oracle.bf16_words_to_f32(oracle.gather(kc, tables[0], 5))
    v = oracle.bf16_words_to_f32(oracle.gather(vc, tables[0], 5))
    bad = np.zeros_like(good)
    for h in range(4):
        s = (k[:, h % 2] @ q.numpy()[0, h]) * scale
        p = np.exp(s - s.max())
        bad[0, h] = (p / p.sum()) @ v[:, h % 2]
    assert not np.allclose(bad, good, atol=1e-3)
