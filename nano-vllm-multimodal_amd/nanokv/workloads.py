"""Seeded synthetic workloads for the paged-KV path.

Five shapes, from the single decode store up to a 28-layer continuous-
batching decode step.  All host-side randomness comes from a CPU
``torch.Generator`` seeded with ``BASE_SEED + index`` (index 0..4 in the
order below; 17 is the reference benchmark's default seed,
nanovllm/benchmark/paged_kv.py:39), so every consumer (device run, CPU
baseline, tests) sees identical metadata and K/V bytes.  Block lists are
built the way the reference's BlockManager hands them out (distinct blocks
per sequence unless deliberately shared as a prefix,
nanovllm/engine/block_manager.py:159-227), so every store slot is unique.

Cache contents are not generated here: callers fill caches on the device
(the values never influence the data movement) or from a host array.

  decode_store      64 seqs x 1 token, 8x128 rows, cache 1024 x 256
  chunked_prefill   16 seqs in one 8192-token chunk, 8 continuing, cache 4096 x 256
  prefix_gather     32 contexts log-uniform [512, 32768], half sharing 8
                    prefix blocks, cache 8192 x 256
  narrow_rows       2x128 rows, 24 seqs of text + 1..3 image spans of 1296
                    tokens, duplicated-image pairs share their prefix blocks
                    (filled and hashed in an earlier step), cache 16384 x 256
  decode_step       28 layers, 256 live contexts log-uniform [256, 16384],
                    16 evicted + 16 admitted, cache [2, 28, ~4.6k, 256, 8, 128]
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

BASE_SEED = 17
BLOCK_SIZE = 256
IMAGE_SPAN_TOKENS = 1296

WORKLOAD_NAMES = ("decode_store", "chunked_prefill", "prefix_gather", "narrow_rows", "decode_step")


def seed_for(name: str) -> int:
    return BASE_SEED + WORKLOAD_NAMES.index(name)


@dataclass
class Workload:
    """Host-side description of one workload.

    ``block_tables`` are per-sequence lists of physical block ids;
    ``num_tokens``/``num_cached``/``num_scheduled``/``num_prompt`` are the
    Sequence fields of each sequence; ``key``/``value`` (CPU tensors,
    [tokens, heads, dim] or [layers, tokens, heads, dim]) are the rows the
    step stores."""

    name: str
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    block_tables: list[list[int]]
    num_tokens: np.ndarray
    num_cached: np.ndarray
    num_scheduled: np.ndarray
    num_prompt: np.ndarray
    key: torch.Tensor | None = None
    value: torch.Tensor | None = None
    slot_mapping: np.ndarray | None = None
    num_layers: int = 1
    phase: str = "prefill"  # "prefill" or "decode"
    extra: dict = field(default_factory=dict)

    @property
    def row_bytes(self) -> int:
        return self.num_kv_heads * self.head_dim * torch.empty((), dtype=self.dtype).element_size()

    @property
    def num_seqs(self) -> int:
        return len(self.block_tables)

    @property
    def context_lens(self) -> np.ndarray:
        """Rows a gather of each sequence's context reads: num_cached +
        num_scheduled (prefill) or num_tokens (decode)."""
        if self.phase == "decode":
            return self.num_tokens.astype(np.int32)
        return (self.num_cached + self.num_scheduled).astype(np.int32)

    def padded_block_tables(self, width: int | None = None) -> np.ndarray:
        longest = max((len(t) for t in self.block_tables), default=0)
        width = longest if width is None else width
        table = np.full((self.num_seqs, width), -1, dtype=np.int32)
        for i, t in enumerate(self.block_tables):
            table[i, : len(t)] = t
        return table

    def cu_seqlens_k(self) -> np.ndarray:
        lens = self.context_lens.astype(np.int64)
        return np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)

    def csr(self) -> tuple[np.ndarray, np.ndarray]:
        counts = [len(t) for t in self.block_tables]
        offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
        ids = np.array([b for t in self.block_tables for b in t], dtype=np.int32)
        return offsets, ids

    # -------------------------------------------------- algorithmic bytes
    def store_bytes(self, layers: int | None = None) -> int:
        """N_valid rows x (read + write) x (K + V) + 4 B per slot read."""
        assert self.slot_mapping is not None
        layers = self.num_layers if layers is None else layers
        valid = int((self.slot_mapping >= 0).sum())
        return layers * (valid * 4 * self.row_bytes + 4 * int(self.slot_mapping.size))

    def gather_bytes(self, layers: int | None = None) -> int:
        """sum(L) rows x (read + write) x (K + V) + the block ids read for K
        and V + cu_seqlens_k."""
        layers = self.num_layers if layers is None else layers
        lens = self.context_lens.astype(np.int64)
        blocks = int(((lens + self.block_size - 1) // self.block_size).sum())
        return layers * (int(lens.sum()) * 4 * self.row_bytes + 8 * blocks + 4 * (self.num_seqs + 1))


    def cu_seqlens_q(self) -> np.ndarray:
        """Exclusive scan of the new tokens per sequence (prefill)."""
        return np.concatenate([[0], np.cumsum(self.num_scheduled.astype(np.int64))]).astype(np.int32)

    def store_gather_bytes(self, layers: int | None = None) -> int:
        """The fused prefill store + context gather: the store's and the
        gather's bytes, less the new rows the gather would read back from the
        cache (the fused launch writes them to the output from the K/V row it
        already read)."""
        layers = self.num_layers if layers is None else layers
        new_rows = int((self.slot_mapping >= 0).sum())
        return (self.store_bytes(layers=layers) + self.gather_bytes(layers=layers)
                - layers * new_rows * 2 * self.row_bytes)


def _generator(seed: int) -> torch.Generator:
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _randn_rows(g: torch.Generator, shape, dtype) -> torch.Tensor:
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def _log_uniform_ints(g: torch.Generator, n: int, low: int, high: int) -> np.ndarray:
    u = torch.rand(n, generator=g, dtype=torch.float64).numpy()
    values = np.exp(math.log(low) + u * (math.log(high) - math.log(low)))
    return np.clip(np.floor(values).astype(np.int64), low, high)


def _prefill_slots(block_tables, cached, scheduled, block_size) -> np.ndarray:
    parts = []
    for table, start, q in zip(block_tables, cached, scheduled):
        if not table:
            continue
        positions = np.arange(int(start), int(start) + int(q), dtype=np.int64)
        ids = np.asarray(table, dtype=np.int64)
        parts.append(ids[positions // block_size] * block_size + positions % block_size)
    return (np.concatenate(parts) if parts else np.zeros(0, np.int64)).astype(np.int32)


def _blocks_for(tokens: int, block_size: int) -> int:
    return (int(tokens) + block_size - 1) // block_size


# ---------------------------------------------------------------- workloads

def decode_store(*, seed: int | None = None, num_seqs: int = 64, num_blocks: int = 1024,
                 max_position: int = 8191, num_padding: int = 4, heads: int = 8,
                 head_dim: int = 128, block_size: int = BLOCK_SIZE,
                 dtype: torch.dtype = torch.bfloat16) -> Workload:
    """One new token per sequence at a position uniform in [0, max_position];
    slot = block_table[pos // BS]*BS + pos % BS.  Every sequence's last
    block is a distinct entry of a seeded permutation of the free blocks;
    its earlier blocks cycle through the rest of the permutation (only the
    last block is written).  ``num_padding`` random rows get slot -1."""
    g = _generator(seed_for("decode_store") if seed is None else seed)
    perm = torch.randperm(num_blocks, generator=g).numpy()
    positions = torch.randint(0, max_position + 1, (num_seqs,), generator=g).numpy()
    rest = perm[num_seqs:]
    tables, cursor = [], 0
    for i, pos in enumerate(positions):
        n_blocks = int(pos) // block_size + 1
        prefix = [int(rest[(cursor + j) % rest.size]) for j in range(n_blocks - 1)]
        cursor += n_blocks - 1
        tables.append(prefix + [int(perm[i])])
    num_tokens = positions + 1
    slots = np.array([t[-1] * block_size + int(p) % block_size for t, p in zip(tables, positions)],
                     dtype=np.int32)
    padding = torch.randperm(num_seqs, generator=g)[:num_padding].numpy()
    slots[padding] = -1
    key = _randn_rows(g, (num_seqs, heads, head_dim), dtype)
    value = _randn_rows(g, (num_seqs, heads, head_dim), dtype)
    return Workload(
        "decode_store", num_blocks, block_size, heads, head_dim, dtype, tables,
        num_tokens.astype(np.int32), (num_tokens - 1).astype(np.int32),
        np.ones(num_seqs, np.int32), num_tokens.astype(np.int32), key, value, slots,
        phase="decode", extra={"padding_rows": np.sort(padding)},
    )


def chunked_prefill(*, seed: int | None = None, num_seqs: int = 16, chunk_tokens: int = 8192,
                    min_len: int = 128, max_len: int = 4096, continuing: int = 8,
                    max_cached_blocks: int = 8, num_blocks: int = 4096, heads: int = 8,
                    head_dim: int = 128, block_size: int = BLOCK_SIZE,
                    dtype: torch.dtype = torch.bfloat16) -> Workload:
    """Lengths uniform in [min_len, max_len] rescaled to fill one
    ``chunk_tokens`` chunk (remainder to the last sequence); the first
    ``continuing`` sequences already hold k*BS cached tokens (k uniform in
    [1, max_cached_blocks]), like continuation chunks."""
    g = _generator(seed_for("chunked_prefill") if seed is None else seed)
    lens = torch.randint(min_len, max_len + 1, (num_seqs,), generator=g).numpy().astype(np.int64)
    q = np.maximum(1, (lens * chunk_tokens) // lens.sum())
    q[-1] += chunk_tokens - q.sum()
    assert q[-1] > 0 and q.sum() == chunk_tokens
    cached = np.zeros(num_seqs, np.int64)
    k = torch.randint(1, max_cached_blocks + 1, (continuing,), generator=g).numpy()
    cached[:continuing] = k * block_size
    perm = torch.randperm(num_blocks, generator=g).numpy()
    tables, cursor = [], 0
    for i in range(num_seqs):
        n = _blocks_for(cached[i] + q[i], block_size)
        tables.append([int(b) for b in perm[cursor : cursor + n]])
        cursor += n
    assert cursor <= num_blocks
    ends = cached + q
    slots = _prefill_slots(tables, cached, q, block_size)
    key = _randn_rows(g, (chunk_tokens, heads, head_dim), dtype)
    value = _randn_rows(g, (chunk_tokens, heads, head_dim), dtype)
    return Workload(
        "chunked_prefill", num_blocks, block_size, heads, head_dim, dtype, tables,
        ends.astype(np.int32), cached.astype(np.int32), q.astype(np.int32),
        ends.astype(np.int32), key, value, slots,
    )


def prefix_gather(*, seed: int | None = None, num_seqs: int = 32, min_ctx: int = 512,
                  max_ctx: int = 32768, shared_blocks: int = 8, num_blocks: int = 8192,
                  heads: int = 8, head_dim: int = 128, block_size: int = BLOCK_SIZE,
                  dtype: torch.dtype = torch.bfloat16) -> Workload:
    """Contexts log-uniform in [min_ctx, max_ctx]; the even-indexed
    sequences share their first ``shared_blocks`` physical blocks (a
    ref-counted prefix), the rest of every table is private."""
    g = _generator(seed_for("prefix_gather") if seed is None else seed)
    ctx = _log_uniform_ints(g, num_seqs, min_ctx, max_ctx)
    perm = torch.randperm(num_blocks, generator=g).numpy()
    shared = [int(b) for b in perm[:shared_blocks]]
    tables, cursor = [], shared_blocks
    for i in range(num_seqs):
        n = _blocks_for(ctx[i], block_size)
        if i % 2 == 0:
            own = min(n, shared_blocks)
            table = shared[:own] + [int(b) for b in perm[cursor : cursor + n - own]]
            cursor += n - own
        else:
            table = [int(b) for b in perm[cursor : cursor + n]]
            cursor += n
        tables.append(table)
    assert cursor <= num_blocks
    zeros = np.zeros(num_seqs, np.int32)
    return Workload(
        "prefix_gather", num_blocks, block_size, heads, head_dim, dtype, tables,
        ctx.astype(np.int32), ctx.astype(np.int32), zeros, ctx.astype(np.int32),
        extra={"shared_prefix_blocks": shared},
    )


NARROW_ROWS_SCHEDULES = ("reference", "same_step")


def narrow_rows(*, seed: int | None = None, num_seqs: int = 24, num_blocks: int = 16384,
                min_text: int = 16, max_text: int = 256, max_images: int = 3,
                image_tokens: int = IMAGE_SPAN_TOKENS, heads: int = 2, head_dim: int = 128,
                block_size: int = BLOCK_SIZE, dtype: torch.dtype = torch.bfloat16,
                schedule: str = "reference") -> Workload:
    """Qwen2.5-VL-3B rows (2 x 128 bf16 = 512 B).  Each sequence is text
    segments (uniform in [min_text, max_text]) interleaved with 1..max_images
    image spans.  Sequence 2k+1 duplicates sequence 2k's prompt up to and
    including its first image, and reuses the full blocks of that prefix
    (prefix-cache reuse is by full blocks chained from block 0,
    block_manager.py:119-198).  The step is a prefill store of every
    non-cached token followed by a gather of every full context.

    ``schedule`` says when the shared blocks were filled:

    * ``"reference"`` — in an earlier step, the only order the reference
      produces: a block is hashed for reuse after the step that wrote it
      (Scheduler.postprocess -> hash_blocks, scheduler.py:196-200,
      block_manager.py:229-258).  Sequence 2k's first chunk prefilled its
      first ``share`` full blocks, which were hashed; in this step 2k
      continues from them and 2k+1 hits the same blocks, so both hold
      share * block_size cached tokens and the step writes none of the
      shared rows.
    * ``"same_step"`` — 2k fills the blocks in this step and 2k+1 reads them
      as its cached prefix.  The reference never schedules this; it is kept
      as an extension for store-then-gather, which handles it."""
    if schedule not in NARROW_ROWS_SCHEDULES:
        raise ValueError(f"schedule must be one of {NARROW_ROWS_SCHEDULES}")
    g = _generator(seed_for("narrow_rows") if seed is None else seed)
    perm = torch.randperm(num_blocks, generator=g).numpy()
    cursor = 0
    tables, totals, cached = [], [], []
    partner_first_text = 0
    for i in range(num_seqs):
        n_images = int(torch.randint(1, max_images + 1, (1,), generator=g))
        texts = torch.randint(min_text, max_text + 1, (n_images + 1,), generator=g).numpy()
        if i % 2 == 1:
            texts[0] = partner_first_text
        total = int(texts.sum()) + n_images * image_tokens
        n = _blocks_for(total, block_size)
        if i % 2 == 1:
            prefix_tokens = int(texts[0]) + image_tokens
            share = min(prefix_tokens // block_size, n - 1, len(tables[-1]))
            table = tables[-1][:share] + [int(b) for b in perm[cursor : cursor + n - share]]
            cursor += n - share
            cached.append(share * block_size)
            if schedule == "reference":
                # the partner's earlier chunk ended at the shared full blocks
                # (it has text after its first image, so it still has new tokens)
                assert share * block_size < totals[-1]
                cached[-2] = share * block_size
        else:
            partner_first_text = int(texts[0])
            table = [int(b) for b in perm[cursor : cursor + n]]
            cursor += n
            cached.append(0)
        tables.append(table)
        totals.append(total)
    assert cursor <= num_blocks
    totals = np.array(totals, np.int64)
    cached = np.array(cached, np.int64)
    scheduled = totals - cached
    slots = _prefill_slots(tables, cached, scheduled, block_size)
    t = int(scheduled.sum())
    key = _randn_rows(g, (t, heads, head_dim), dtype)
    value = _randn_rows(g, (t, heads, head_dim), dtype)
    return Workload(
        "narrow_rows", num_blocks, block_size, heads, head_dim, dtype, tables,
        totals.astype(np.int32), cached.astype(np.int32), scheduled.astype(np.int32),
        totals.astype(np.int32), key, value, slots, extra={"schedule": schedule},
    )


def decode_step(*, seed: int | None = None, num_layers: int = 28, num_live: int = 256,
                churn: int = 16, min_ctx: int = 256, max_ctx: int = 16384, heads: int = 8,
                head_dim: int = 128, block_size: int = BLOCK_SIZE, headroom: float = 0.10,
                dtype: torch.dtype = torch.bfloat16) -> Workload:
    """A continuous-batching decode step.  ``num_live`` sequences with
    contexts log-uniform in [min_ctx, max_ctx] hold blocks from a seeded
    free list; ``churn`` of them finish and return their blocks to the
    front of the free list; ``churn`` admitted requests (same context law)
    take fresh block lists from it.  The step decodes one token for each
    of the resulting ``num_live`` sequences (the context includes it), in
    every one of ``num_layers`` layers.  The pool holds the blocks in use at
    the peak plus ``headroom``."""
    g = _generator(seed_for("decode_step") if seed is None else seed)
    ctx = _log_uniform_ints(g, num_live, min_ctx, max_ctx)
    admitted_ctx = _log_uniform_ints(g, churn, min_ctx, max_ctx)
    evicted = np.sort(torch.randperm(num_live, generator=g)[:churn].numpy())
    need = np.array([_blocks_for(c, block_size) for c in ctx])
    need_admit = np.array([_blocks_for(c, block_size) for c in admitted_ctx])
    peak = int(need.sum()) + max(0, int(need_admit.sum()) - int(need[evicted].sum()))
    num_blocks = int(math.ceil(peak * (1.0 + headroom) / 64.0) * 64)
    free = list(torch.randperm(num_blocks, generator=g).numpy().tolist())
    tables = []
    for n in need:
        tables.append(free[:n])
        del free[:n]
    freed = [b for i in evicted for b in tables[i]]
    free = freed + free
    gone = set(evicted.tolist())
    survivors = [i for i in range(num_live) if i not in gone]
    live_tables = [tables[i] for i in survivors]
    live_ctx = [int(ctx[i]) for i in survivors]
    for c, n in zip(admitted_ctx, need_admit):
        live_tables.append(free[:n])
        del free[:n]
        live_ctx.append(int(c))
    num_tokens = np.array(live_ctx, np.int32)
    last = num_tokens.astype(np.int64) - 1
    slots = np.array(
        [t[p // block_size] * block_size + p % block_size for t, p in zip(live_tables, last)],
        dtype=np.int32,
    )
    key = _randn_rows(g, (num_layers, num_live, heads, head_dim), dtype)
    value = _randn_rows(g, (num_layers, num_live, heads, head_dim), dtype)
    return Workload(
        "decode_step", num_blocks, block_size, heads, head_dim, dtype, live_tables,
        num_tokens, (num_tokens - 1).astype(np.int32), np.ones(num_live, np.int32), num_tokens,
        key, value, slots, num_layers=num_layers, phase="decode",
        extra={"evicted": evicted, "admitted": churn},
    )


BUILDERS = {
    "decode_store": decode_store,
    "chunked_prefill": chunked_prefill,
    "prefix_gather": prefix_gather,
    "narrow_rows": narrow_rows,
    "decode_step": decode_step,
}


def build(name: str, **overrides) -> Workload:
    return BUILDERS[name](**overrides)
