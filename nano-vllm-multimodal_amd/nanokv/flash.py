"""Drop-ins for the two flash-attn calls of the reference's Attention.forward
(nanovllm/layers/attention.py:5 imports them; :105-116 prefill, :122-130
decode), run by the hip paged-attention kernels on the paged KV cache.  A
ROCm build of the engine replaces ``from flash_attn import
flash_attn_varlen_func, flash_attn_with_kvcache`` with an import from this
module; the calls stay as they are.

Only what the reference passes is supported: causal attention, bfloat16 or
float16, head_dim 128, 1 to 8 query heads per kv head for prefill (1, 2, 4
or 8 kv heads) and 1 to 16 for decode, no dropout, window, alibi or
softcap.  Anything else raises instead of computing something
different.
"""
from __future__ import annotations

import math
import threading
import weakref

import torch

from nanokv.paged_kv.base import index_value_validation_enabled
from nanokv.paged_kv.hip_backend import HIPPagedKVBackend

_BACKEND = HIPPagedKVBackend()
_UNSUPPORTED_DEFAULTS = {
    "dropout_p": 0.0,
    "window_size": (-1, -1),
    "softcap": 0.0,
    "alibi_slopes": None,
    "deterministic": False,
    "return_attn_probs": False,
}


def _check_options(name: str, causal: bool, options: dict) -> None:
    if not causal:
        raise NotImplementedError(f"{name}: only causal attention is implemented "
                                  "(the reference always passes causal=True)")
    for key, value in options.items():
        if key not in _UNSUPPORTED_DEFAULTS:
            raise TypeError(f"{name}: unexpected argument {key!r}")
        if value != _UNSUPPORTED_DEFAULTS[key]:
            raise NotImplementedError(f"{name}: {key}={value!r} is not supported")


def flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k, cu_seqlens_k,
                           softmax_scale=None, causal=False, block_table=None, **options):
    """Causal varlen attention (attention.py:105-116).  With ``block_table``
    k and v are the paged caches [blocks, block_size, kv_heads, 128] and
    request i reads the first cu_seqlens_k[i+1] - cu_seqlens_k[i] rows of its
    table; without, k and v hold every request's keys back to back
    [total_k, kv_heads, 128].  The queries of a request are the last ones of
    its context (bottom-right causal alignment).  Returns [total_q, heads, 128]."""
    _check_options("flash_attn_varlen_func", causal, options)
    scale = 1.0 / math.sqrt(q.shape[-1]) if softmax_scale is None else float(softmax_scale)
    if block_table is None:
        # Contiguous keys: a cache of one-row blocks whose table for request
        # i counts up from cu_seqlens_k[i] (entries past its length are
        # never read).
        if k.ndim != 3 or v.shape != k.shape:
            raise ValueError("without block_table, k and v must be [total_k, kv_heads, head_dim]")
        k_cache = k.contiguous().unsqueeze(1)
        v_cache = v.contiguous().unsqueeze(1)
        width = max(1, int(max_seqlen_k))
        columns = torch.arange(width, dtype=torch.int32, device=k.device)
        block_table = (cu_seqlens_k[:-1].unsqueeze(1) + columns.unsqueeze(0)).contiguous()
    else:
        k_cache, v_cache = k, v
    return _BACKEND.paged_attention_prefill(q, k_cache, v_cache, block_table, cu_seqlens_q,
                                            cu_seqlens_k, scale)


class _StepPlan:
    """The decode plan of the current step.  Every layer of a step passes the
    same cache_seqlens tensor and its own cache, so the first call reads the
    context total back once and builds the plan, and the step's other layers
    reuse both.  The entry holds while the same tensor object comes back
    (a weak reference) with the same shape, device and block size, and, where
    torch tracks it, the same version (an in-place update, or the device
    packer's writes, which bump it).  A layer's cache seen a second time
    starts a new step and a new plan: this covers inference tensors
    (torch.inference_mode), which carry no version counter."""

    def __init__(self) -> None:
        self._lock = threading.Lock()
        self._entry = None  # [weakref to cache_seqlens, key, cu_seqlens_k, total, plan, caches seen]

    def lookup(self, cache_seqlens, key, cache_ptr: int):
        with self._lock:
            entry = self._entry
            if (entry is None or entry[0]() is not cache_seqlens or entry[1] != key
                    or cache_ptr in entry[5]):
                return None
            entry[5].add(cache_ptr)
            return entry[2], entry[3], entry[4]

    def store(self, cache_seqlens, key, cache_ptr: int, cu_seqlens_k, total, plan) -> None:
        with self._lock:
            self._entry = [weakref.ref(cache_seqlens), key, cu_seqlens_k, total, plan, {cache_ptr}]


_STEP_PLAN = _StepPlan()


def flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=None, block_table=None,
                            softmax_scale=None, causal=False, **options):
    """One decode token per sequence over its paged context
    (attention.py:122-130): q [batch, 1, heads, 128], caches [blocks,
    block_size, kv_heads, 128], cache_seqlens [batch] int32 context lengths,
    block_table [batch, width] int32.  Returns [batch, 1, heads, 128].

    Outside graph capture the first call of a step reads the total context
    length back (one synchronisation per step, not per layer) and builds a
    plan of exactly the context's entries, which the step's other layers
    reuse (see _StepPlan for what ends a step).  Under graph capture nothing may be read back: the plan is then
    sized for the longest contexts the tables can hold (batch x width x
    block_size rows), and its padding entries cost workgroups that exit at
    once."""
    _check_options("flash_attn_with_kvcache", causal, options)
    if q.ndim != 4 or q.shape[1] != 1:
        raise NotImplementedError("flash_attn_with_kvcache: one query token per sequence only")
    if cache_seqlens is None or block_table is None:
        raise NotImplementedError("flash_attn_with_kvcache: needs cache_seqlens and block_table")
    scale = 1.0 / math.sqrt(q.shape[-1]) if softmax_scale is None else float(softmax_scale)
    batch = q.shape[0]
    capturing = torch.cuda.is_current_stream_capturing()
    version = None if cache_seqlens.is_inference() else cache_seqlens._version
    key = (cache_seqlens.data_ptr(), version, tuple(cache_seqlens.shape), str(q.device),
           int(k_cache.shape[1]), int(k_cache.shape[2]))
    cache_ptr = k_cache.data_ptr()
    cached = None if capturing else _STEP_PLAN.lookup(cache_seqlens, key, cache_ptr)
    if cached is not None:
        cu_seqlens_k, total, plan = cached
    else:
        lengths = cache_seqlens.to(device=q.device, dtype=torch.int32)
        cu_seqlens_k = torch.zeros(batch + 1, dtype=torch.int32, device=q.device)
        torch.cumsum(lengths, 0, out=cu_seqlens_k[1:])
        if capturing and not index_value_validation_enabled(lengths):
            total = batch * block_table.shape[1] * k_cache.shape[1]
            plan = None
        else:
            total = int(cu_seqlens_k[-1])
            plan = _BACKEND.build_attention_plan(k_cache, cu_seqlens_k, total)
            if not capturing:
                _STEP_PLAN.store(cache_seqlens, key, cache_ptr, cu_seqlens_k, total, plan)
    out = _BACKEND.paged_attention_decode(q[:, 0], k_cache, v_cache, block_table, cu_seqlens_k,
                                          total, scale, plan=plan)
    return out.unsqueeze(1)
