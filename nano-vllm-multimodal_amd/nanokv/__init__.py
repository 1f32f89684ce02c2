"""nanokv: NanoInfer's paged KV store / gather hot path and its ragged-batch
metadata packing, as hand-written HIP kernels for AMD Instinct MI355X
(gfx950), behind the reference's ``paged_kv_backend`` plugin API as the
``hip`` backend.

Layout:
  nanokv.paged_kv   backend protocol, validators, name resolution, the
                    ``hip`` backend and the ``nanovllm_paged_kv`` op
                    registration
  nanokv.packing    device-side packing of cu_seqlens / slot_mapping /
                    block_tables from per-sequence scheduler state
  nanokv.workloads  seeded synthetic workloads (decode store, chunked
                    prefill, prefix-cache gather, narrow rows, decode step)
  nanokv.benchmark  timing, byte accounting and percentiles
  nanokv.build      hipcc build of libnanokv.so (C ABI: include/nanokv.h)
"""
from __future__ import annotations

__version__ = "0.1.0"
