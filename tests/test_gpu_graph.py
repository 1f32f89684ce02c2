"""Graph-stable decode metadata on the GPU.

pack_decode_into writes the step's metadata straight into the fixed
buffers a captured decode graph reads, reproducing the reference's replay
fill (model_runner.py:993-1011, restated as oracle.graph_replay_fill):
slot -1 and context length 0 past the batch, block_tables[:bs, :w]
rewritten, stale columns and rows kept.  A graph of plan + per-layer store
+ planned varlen gather is captured once and replayed for several batches,
with eager packing between replays, every replay checked against the
oracle (no memset is recorded in the graph).  So is the Flash path's graph
decode: per-layer store + the flash_attn_with_kvcache drop-in.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv as oracle

pytestmark = pytest.mark.gpu

BS = 16
HEADS, DIM = 2, 64


def random_batch(rng, num_seqs, max_tokens, num_blocks):
    n = rng.integers(1, max_tokens + 1, num_seqs)
    need = (n + BS - 1) // BS
    perm = rng.permutation(num_blocks)
    offsets = np.concatenate([[0], np.cumsum(need)])
    assert offsets[-1] <= num_blocks
    tables = [perm[offsets[i]:offsets[i + 1]].tolist() for i in range(num_seqs)]
    return n, tables


def test_pack_decode_into_reproduces_replay_fill(gpu_device):
    from nanokv.packing import DecodeGraphBuffers, DevicePacker, SequenceBatch

    rng = np.random.default_rng(0)
    buffers = DecodeGraphBuffers.allocate(gpu_device, max_num_seqs=24, max_blocks=12)
    for t in (buffers.slot_mapping, buffers.context_lens, buffers.block_tables, buffers.cu_seqlens_k):
        t.fill_(77)
    host = {k: getattr(buffers, k).cpu().numpy().copy() for k in ("slot_mapping", "context_lens", "block_tables")}
    packer = DevicePacker(gpu_device, BS)
    for num_seqs, max_tokens in ((20, 12 * BS), (7, 3 * BS), (24, 5 * BS), (1, 1)):
        n, tables = random_batch(rng, num_seqs, max_tokens, 600)
        ctx = packer.pack_decode_into(SequenceBatch.from_block_lists(n, tables), buffers)
        seqs = [oracle.SeqState(int(n[i]), tables[i]) for i in range(num_seqs)]
        exp = oracle.prepare_decode(seqs, BS)
        oracle.graph_replay_fill(host, exp["slot_mapping"], exp["context_lens"], exp["block_tables"])
        for key in ("slot_mapping", "context_lens", "block_tables"):
            np.testing.assert_array_equal(getattr(buffers, key).cpu().numpy(), host[key], err_msg=key)
        cu = buffers.cu_seqlens_k.cpu().numpy()
        np.testing.assert_array_equal(cu[: num_seqs + 1], exp["cu_seqlens_k"])
        assert (cu[num_seqs + 1:] == exp["cu_seqlens_k"][-1]).all()
        assert ctx.total_context_tokens == int(n.sum())
        np.testing.assert_array_equal(ctx.slot_mapping.cpu().numpy(), exp["slot_mapping"])


def test_captured_decode_graph_replays_match_oracle(gpu_device):
    from nanokv.packing import DecodeGraphBuffers, DevicePacker, SequenceBatch
    from nanokv.paged_kv import create_paged_kv_backend

    backend = create_paged_kv_backend("hip")
    rng = np.random.default_rng(1)
    layers, bucket, max_blocks, num_blocks = 2, 8, 6, 64
    shape = (2, layers, num_blocks, BS, HEADS, DIM)
    cache = torch.randn(shape, dtype=torch.float32, device=gpu_device).to(torch.bfloat16)
    buffers = DecodeGraphBuffers.allocate(gpu_device, max_num_seqs=bucket, max_blocks=max_blocks)
    packer = DevicePacker(gpu_device, BS)
    max_rows = bucket * max_blocks * BS
    key_in = torch.zeros((layers, bucket, HEADS, DIM), dtype=torch.bfloat16, device=gpu_device)
    value_in = torch.zeros_like(key_in)
    k_out = torch.zeros((max_rows, HEADS, DIM), dtype=torch.bfloat16, device=gpu_device)
    v_out = torch.zeros_like(k_out)

    # First batch: eager pack, eager warmup of the captured work, capture.
    n, tables = random_batch(rng, bucket, max_blocks * BS, num_blocks)
    packer.pack_decode_into(SequenceBatch.from_block_lists(n, tables), buffers)

    def decode_work():
        plan = backend.build_gather_plan(cache[0, 0], buffers.block_tables, buffers.cu_seqlens_k, max_rows)
        for layer in range(layers):
            kc, vc = cache[0, layer], cache[1, layer]
            backend.store(key_in[layer], value_in[layer], kc, vc, buffers.slot_mapping)
            backend.gather_varlen(kc, vc, buffers.block_tables, buffers.cu_seqlens_k, max_rows,
                                  plan=plan, out=(k_out, v_out))
        return plan

    decode_work()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan_keepalive = decode_work()
    torch.cuda.synchronize()

    host = cache.cpu().view(torch.int16).numpy().copy()
    for replay in range(4):
        num_seqs = int(rng.integers(1, bucket + 1))
        n, tables = random_batch(rng, num_seqs, max_blocks * BS, num_blocks)
        ctx = packer.pack_decode_into(SequenceBatch.from_block_lists(n, tables), buffers)
        key_in.copy_(torch.randn(key_in.shape, device=gpu_device).to(torch.bfloat16))
        value_in.copy_(torch.randn(value_in.shape, device=gpu_device).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        slots = ctx.slot_mapping.cpu().numpy()
        padded_slots = np.concatenate([slots, np.full(bucket - num_seqs, -1, np.int32)])
        seqs = [oracle.SeqState(int(n[i]), tables[i]) for i in range(num_seqs)]
        exp = oracle.prepare_decode(seqs, BS)
        np.testing.assert_array_equal(slots, exp["slot_mapping"])
        total = int(n.sum())
        for layer in range(layers):
            hk, hv = host[0, layer], host[1, layer]
            oracle.store(key_in[layer].cpu().view(torch.int16).numpy(),
                         value_in[layer].cpu().view(torch.int16).numpy(), hk, hv, padded_slots)
        np.testing.assert_array_equal(cache.cpu().view(torch.int16).numpy(), host, err_msg=f"replay {replay}")
        # The last layer's gather is what the outputs hold after the replay.
        last = layers - 1
        np.testing.assert_array_equal(
            k_out[:total].cpu().view(torch.int16).numpy(),
            oracle.gather_varlen(host[0, last], exp["block_tables"], n), err_msg=f"replay {replay} K")
        np.testing.assert_array_equal(
            v_out[:total].cpu().view(torch.int16).numpy(),
            oracle.gather_varlen(host[1, last], exp["block_tables"], n), err_msg=f"replay {replay} V")
    del plan_keepalive


@pytest.mark.parametrize("kv_heads,q_heads", [(8, 16), (2, 16)])
def test_captured_flash_decode_replays_match_oracle(gpu_device, kv_heads, q_heads):
    """The reference's graph decode on the Flash path (model_runner.py:
    1079-1157 captures Attention.forward; attention.py:87-93 store,
    :122-130 flash_attn_with_kvcache), with the drop-in from nanokv.flash:
    per layer, store then decode attention over the paged cache, captured
    once and replayed for batches of 1..bucket sequences (padding rows have
    context length 0; the attention plan is built inside the graph, so
    each replay splits its own lengths).  Every replay's cache is checked
    bit for bit and its attention output within 1e-3 + 2^-8 (ref_abs +
    |ref|) against the oracle (ref_abs: the same attention over |V|; the
    kernel rounds its weights to bf16)."""
    from nanokv.flash import flash_attn_with_kvcache
    from nanokv.packing import DecodeGraphBuffers, DevicePacker, SequenceBatch
    from nanokv.paged_kv import create_paged_kv_backend

    backend = create_paged_kv_backend("hip")
    rng = np.random.default_rng(3)
    layers, bucket, max_blocks, num_blocks, dim = 2, 8, 6, 64, 128
    scale = 1.0 / np.sqrt(dim)
    shape = (2, layers, num_blocks, BS, kv_heads, dim)
    cache = torch.randn(shape, dtype=torch.float32, device=gpu_device).to(torch.bfloat16)
    buffers = DecodeGraphBuffers.allocate(gpu_device, max_num_seqs=bucket, max_blocks=max_blocks)
    packer = DevicePacker(gpu_device, BS)
    key_in = torch.zeros((layers, bucket, kv_heads, dim), dtype=torch.bfloat16, device=gpu_device)
    value_in = torch.zeros_like(key_in)
    q_in = torch.zeros((bucket, q_heads, dim), dtype=torch.bfloat16, device=gpu_device)

    n, tables = random_batch(rng, bucket, max_blocks * BS, num_blocks)
    packer.pack_decode_into(SequenceBatch.from_block_lists(n, tables), buffers)

    def decode_work():
        outs = []
        for layer in range(layers):
            kc, vc = cache[0, layer], cache[1, layer]
            backend.store(key_in[layer], value_in[layer], kc, vc, buffers.slot_mapping)
            outs.append(flash_attn_with_kvcache(q_in.unsqueeze(1), kc, vc,
                                                cache_seqlens=buffers.context_lens,
                                                block_table=buffers.block_tables,
                                                softmax_scale=scale, causal=True))
        return outs

    decode_work()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = decode_work()
    torch.cuda.synchronize()

    host = cache.cpu().view(torch.int16).numpy().copy()
    for replay in range(4):
        num_seqs = int(rng.integers(1, bucket + 1))
        n, tables = random_batch(rng, num_seqs, max_blocks * BS, num_blocks)
        ctx = packer.pack_decode_into(SequenceBatch.from_block_lists(n, tables), buffers)
        key_in.copy_(torch.randn(key_in.shape, device=gpu_device).to(torch.bfloat16))
        value_in.copy_(torch.randn(value_in.shape, device=gpu_device).to(torch.bfloat16))
        q_in.copy_(torch.randn(q_in.shape, device=gpu_device).to(torch.bfloat16))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        slots = ctx.slot_mapping.cpu().numpy()
        padded_slots = np.concatenate([slots, np.full(bucket - num_seqs, -1, np.int32)])
        seqs = [oracle.SeqState(int(n[i]), tables[i]) for i in range(num_seqs)]
        exp = oracle.prepare_decode(seqs, BS)
        q_host = q_in[:num_seqs].float().cpu().numpy()
        for layer in range(layers):
            hk, hv = host[0, layer], host[1, layer]
            oracle.store(key_in[layer].cpu().view(torch.int16).numpy(),
                         value_in[layer].cpu().view(torch.int16).numpy(), hk, hv, padded_slots)
            ref = oracle.paged_attention_decode(q_host, hk, hv, exp["block_tables"], n, scale)
            ref_abs = oracle.paged_attention_decode(q_host, hk, hv & np.int16(0x7FFF),
                                                    exp["block_tables"], n, scale)
            got = outs[layer][:, 0].float().cpu().numpy()
            bad = np.abs(got[:num_seqs] - ref) > 1e-3 + 2.0 ** -8 * (ref_abs + np.abs(ref))
            assert not bad.any(), f"replay {replay} layer {layer}: {int(bad.sum())} elements off"
            assert not got[num_seqs:].any(), f"replay {replay} layer {layer}: padding rows not zero"
        np.testing.assert_array_equal(cache.cpu().view(torch.int16).numpy(), host,
                                      err_msg=f"replay {replay}")
