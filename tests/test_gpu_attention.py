"""Paged-attention decode on the GPU vs the float32 oracle
(oracle.paged_kv.paged_attention_decode, itself pinned to torch's SDPA with
GQA in tests/test_attention_oracle.py).

Tolerance: the kernel accumulates in fp32 and rounds the result to bf16
once, so every element must satisfy |hip - ref| <= 1e-3 + 1e-2 * |ref|
(bf16 rounding is <= 2^-9 relative; fp32 summation-order and exp2 error
are orders of magnitude smaller).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_kv as oracle

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-2


@pytest.fixture(scope="module")
def backend(gpu_device):
    from nanokv.paged_kv import create_paged_kv_backend

    return create_paged_kv_backend("hip")


def check_close(got: torch.Tensor, ref: np.ndarray, what: str) -> None:
    g = got.float().cpu().numpy()
    bad = np.abs(g - ref) > ATOL + RTOL * np.abs(ref)
    assert not bad.any(), f"{what}: {int(bad.sum())} elements off, max err {np.abs(g - ref).max():.3e}"


def build_case(device, hkv, g, bs, lens, seed, q_pad_heads=0):
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
    kc = torch.randn(nb, bs, hkv, 128, generator=gen).to(torch.bfloat16)
    vc = torch.randn(nb, bs, hkv, 128, generator=gen).to(torch.bfloat16)
    hq = hkv * g
    q_full = torch.randn(b, hq + q_pad_heads, 128, generator=gen).to(torch.bfloat16)
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
])
def test_decode_attention_matches_oracle(backend, gpu_device, hkv, g, bs):
    lens = [0, 1, bs - 1, bs, bs + 1, 3 * bs + 7, 2, 5 * bs, 17, 1]
    dev, host, total = build_case(gpu_device, hkv, g, bs, lens, seed=hkv * 100 + g * 10 + bs)
    scale = 1.0 / math.sqrt(128)
    out = backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                         total, scale)
    ref = oracle.paged_attention_decode(host["q"], host["kc"], host["vc"], host["tables"],
                                        host["lens"], scale)
    check_close(out, ref, f"hkv={hkv} g={g} bs={bs}")
    assert torch.all(out[0] == 0), "an empty context must give zeros"


def test_strided_q_plan_reuse_and_out_buffer(backend, gpu_device):
    lens = [300, 1, 513, 256, 40]
    dev, host, total = build_case(gpu_device, 8, 2, 256, lens, seed=7, q_pad_heads=16)
    assert dev["q"].stride(0) == 32 * 128
    plan = backend.build_attention_plan(dev["kc"], dev["tables"], dev["cu"], total)
    out = torch.empty((len(lens), 16, 128), dtype=torch.bfloat16, device=gpu_device)
    ref = oracle.paged_attention_decode(host["q"], host["kc"], host["vc"], host["tables"],
                                        host["lens"], 0.1)
    for _ in range(2):
        out.zero_()
        backend.paged_attention_decode(dev["q"], dev["kc"], dev["vc"], dev["tables"], dev["cu"],
                                       total, 0.1, plan=plan, out=out)
        check_close(out, ref, "planned")


def test_decode_step_layer_full_size(backend, gpu_device):
    """One layer of the 256-sequence decode step (contexts log-uniform in
    [256, 16384], 8 kv heads x 2 query heads each), every element checked."""
    from nanokv import workloads

    wl = workloads.build("decode_step", num_layers=1)
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    gen = torch.Generator(device=gpu_device).manual_seed(3)
    kc = torch.randn(shape, device=gpu_device, generator=gen).to(torch.bfloat16)
    vc = torch.randn(shape, device=gpu_device, generator=gen).to(torch.bfloat16)
    q = torch.randn((wl.num_seqs, 16, 128), device=gpu_device, generator=gen).to(torch.bfloat16)
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
    ref = oracle.paged_attention_decode(q.float().cpu().numpy(), hk, hv, ctables, wl.num_tokens,
                                        1 / math.sqrt(128))
    check_close(out, ref, "decode step layer")
