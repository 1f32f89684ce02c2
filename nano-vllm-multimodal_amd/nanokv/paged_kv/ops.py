"""``torch.library`` registration of the paged-KV ops, implemented by the
HIP library through its C ABI.

Namespace and the two reference schemas are unchanged
(csrc/paged_kv/paged_kv.cpp:199-203):

    nanovllm_paged_kv::store(Tensor key, Tensor value, Tensor(a!) key_cache,
                             Tensor(b!) value_cache, Tensor slot_mapping) -> ()
    nanovllm_paged_kv::gather(Tensor cache, Tensor block_table,
                              int sequence_length) -> Tensor

The implementations sit on the CUDA dispatch key, the key ROCm device
tensors carry under PyTorch-ROCm (the reference registers its kernels there
too, paged_kv_cuda.cu:168-171).  Additive ops, with no reference schema:

    gather_varlen(Tensor key_cache, Tensor value_cache, Tensor block_tables,
                  Tensor cu_seqlens_k, int total_tokens) -> (Tensor, Tensor)
    build_gather_plan(Tensor block_tables, Tensor cu_seqlens_k,
                      int total_tokens, int num_blocks, int block_size,
                      int row_elems, ScalarType dtype) -> Tensor
    gather_varlen_planned(Tensor key_cache, Tensor value_cache, Tensor plan,
                          Tensor(a!) key_out, Tensor(b!) value_out) -> ()
    build_attention_plan(Tensor cu_seqlens_k, int total_tokens,
                         int block_size, int num_kv_heads) -> (Tensor, Tensor)
    paged_attention_decode(Tensor q, Tensor key_cache, Tensor value_cache,
                           Tensor block_tables, Tensor plan,
                           Tensor first_part, float scale,
                           Tensor(a!) out) -> ()
    build_store_gather_plan(Tensor block_tables, Tensor cu_seqlens_q,
                            Tensor cu_seqlens_k, int num_tokens,
                            int total_tokens, int num_blocks, int block_size,
                            int row_elems, ScalarType dtype) -> Tensor
    store_gather(Tensor key, Tensor value, Tensor(a!) key_cache,
                 Tensor(b!) value_cache, Tensor slot_mapping, Tensor plan,
                 int num_seqs, Tensor(c!) key_out, Tensor(d!) value_out) -> ()

Every kernel runs on the current stream of the tensors' device and returns
before it completes, like the reference ops.
"""
from __future__ import annotations

from threading import Lock

import torch

from nanokv import _lib

NAMESPACE = "nanovllm_paged_kv"

SCHEMAS = {
    "store": "store(Tensor key, Tensor value, Tensor(a!) key_cache, "
    "Tensor(b!) value_cache, Tensor slot_mapping) -> ()",
    "gather": "gather(Tensor cache, Tensor block_table, int sequence_length) -> Tensor",
    "gather_varlen": "gather_varlen(Tensor key_cache, Tensor value_cache, "
    "Tensor block_tables, Tensor cu_seqlens_k, int total_tokens) -> (Tensor, Tensor)",
    "build_gather_plan": "build_gather_plan(Tensor block_tables, Tensor cu_seqlens_k, "
    "int total_tokens, int num_blocks, int block_size, int row_elems, "
    "ScalarType dtype) -> Tensor",
    "gather_varlen_planned": "gather_varlen_planned(Tensor key_cache, Tensor value_cache, "
    "Tensor plan, Tensor(a!) key_out, Tensor(b!) value_out) -> ()",
    "build_attention_plan": "build_attention_plan(Tensor cu_seqlens_k, int total_tokens, "
    "int block_size, int num_kv_heads) -> (Tensor, Tensor)",
    "paged_attention_decode": "paged_attention_decode(Tensor q, Tensor key_cache, "
    "Tensor value_cache, Tensor block_tables, Tensor plan, Tensor first_part, float scale, "
    "Tensor(a!) out) -> ()",
    "build_store_gather_plan": "build_store_gather_plan(Tensor block_tables, "
    "Tensor cu_seqlens_q, Tensor cu_seqlens_k, int num_tokens, int total_tokens, "
    "int num_blocks, int block_size, int row_elems, ScalarType dtype) -> Tensor",
    "store_gather": "store_gather(Tensor key, Tensor value, Tensor(a!) key_cache, "
    "Tensor(b!) value_cache, Tensor slot_mapping, Tensor plan, int num_seqs, "
    "Tensor(c!) key_out, Tensor(d!) value_out) -> ()",
    "build_prefill_plan": "build_prefill_plan(Tensor cu_seqlens_q, Tensor cu_seqlens_k, "
    "int total_q_tokens, int group) -> Tensor",
    "paged_attention_prefill": "paged_attention_prefill(Tensor q, Tensor key_cache, "
    "Tensor value_cache, Tensor block_tables, Tensor cu_seqlens_q, Tensor cu_seqlens_k, "
    "Tensor plan, float scale, Tensor(a!) out) -> ()",
}

DTYPE_CODES = {
    torch.float16: _lib.NKV_DTYPE_FLOAT16,
    torch.bfloat16: _lib.NKV_DTYPE_BFLOAT16,
    torch.float32: _lib.NKV_DTYPE_FLOAT32,
}

_REGISTER_LOCK = Lock()
_FRAGMENT: torch.library.Library | None = None


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise RuntimeError(
            f"nanokv paged KV ops support float16, bfloat16 and float32, not {dtype}"
        ) from None


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(device: torch.device) -> int:
    """The current stream of ``device`` as a hipStream_t integer: torch's raw
    accessor when it exists (no Stream object per launch, ~0.1 us against
    ~2 us), the public Stream object otherwise."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    if _RAW_STREAM is not None:
        return _RAW_STREAM(index)
    return torch.cuda.current_stream(device).cuda_stream


_stream = current_stream_handle


def _require_device(what: str, *tensors: torch.Tensor) -> torch.device:
    index = tensors[0].get_device()  # -1 for host tensors
    for tensor in tensors:
        if tensor.get_device() != index or not tensor.is_cuda:
            raise ValueError(f"{what} requires ROCm device tensors on one device")
    return tensors[0].device


def _require_contiguous_cache(what: str, *caches: torch.Tensor) -> None:
    for cache in caches:
        if not cache.is_contiguous():
            raise ValueError(f"{what} requires contiguous [blocks, block, kv_heads, head_dim] caches")


def _int32_index(what: str, name: str, index: torch.Tensor) -> torch.Tensor:
    """An index tensor as the kernels read it: int32 (a direct op call with
    another dtype raises, as the reference op's typed data_ptr<int32_t> does)
    and contiguous (a strided view is compacted on the device)."""
    if index.dtype != torch.int32:
        raise RuntimeError(f"{what}: {name} must be int32, got {index.dtype}")
    return index if index.is_contiguous() else index.contiguous()


def _plan_capacity(total: int, num_seqs: int, block_size: int, row_elems: int, code: int) -> int:
    return int(
        _lib.load_library().nkv_gather_plan_capacity(total, num_seqs, block_size, row_elems, code)
    )


def _require_store_rows(key, value, key_cache, value_cache, slot_mapping) -> None:
    """The sizes the store kernel trusts: the row size comes from the
    caches, and one int32 slot is read per key row.  (The reference op
    leaves these to the backend's validator; a direct op call that broke
    them would address rows past the caches or the slot list.)"""
    if (key.ndim != 3 or key.shape != value.shape or key_cache.ndim != 4
            or key_cache.shape != value_cache.shape or key.shape[1:] != key_cache.shape[2:]):
        raise RuntimeError("Paged KV HIP Store: key/value [tokens, kv_heads, head_dim] must match "
                           "each other and the caches' [.., kv_heads, head_dim]")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise RuntimeError("Paged KV HIP Store: key/value inner dimensions must be contiguous")
    if slot_mapping.ndim != 1 or slot_mapping.shape[0] != key.shape[0]:
        raise RuntimeError("Paged KV HIP Store: slot_mapping must hold one slot per token")


def stream_of(index: int) -> int:
    """The current stream of GPU ``index`` as a hipStream_t integer."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(index)
    return torch.cuda.current_stream(index).cuda_stream


def store_checked(key, value, key_cache, value_cache, slot_mapping) -> None:
    """The store launch for inputs that already meet the store contract
    (the backend's validator, or the op's own checks): one GPU, matching
    shapes and dtypes, a contiguous int32 slot_mapping with one slot per
    token.  What remains is what only the kernel needs: contiguous caches,
    a contiguous row per token, a dtype it moves."""
    if not (key_cache.is_contiguous() and value_cache.is_contiguous()):
        raise ValueError("paged KV HIP Store requires contiguous [blocks, block, kv_heads, "
                         "head_dim] caches")
    shape = key.shape
    num_tokens = shape[0]
    if num_tokens == 0:
        return
    code = DTYPE_CODES.get(key.dtype)
    if code is None:
        dtype_code(key.dtype)  # raises with the supported dtypes
    # The kernel addresses a token's [kv_heads, head_dim] as one contiguous
    # row through the token stride.  A head-strided view (e.g. kv[:, :, :128]
    # of a [T, H, 256] tensor) passes the validators, which only require a
    # contiguous last dimension, so it is compacted on the device first.
    kstride = key.stride()
    if shape[1] > 1 and kstride[1] != shape[2]:
        key = key.contiguous()
        kstride = key.stride()
    vstride = value.stride()
    if shape[1] > 1 and vstride[1] != shape[2]:
        value = value.contiguous()
        vstride = value.stride()
    cshape = key_cache.shape
    status = _lib.load_library().nkv_store(
        key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
        slot_mapping.data_ptr(), num_tokens, kstride[0], vstride[0], shape[1] * shape[2],
        cshape[0] * cshape[1], code, stream_of(key.get_device()),
    )
    if status:
        _lib.check(status, "nanovllm_paged_kv::store")


def gather_checked(cache, block_table, sequence_length: int) -> torch.Tensor:
    """The gather launch for inputs that already meet the gather contract
    (a 4-D cache and a contiguous 1-D int32 table on one GPU, covering the
    length).  Returns a new [sequence_length, kv_heads, head_dim] tensor of
    the cache's dtype on its device."""
    if not cache.is_contiguous():
        raise ValueError("paged KV HIP Gather requires contiguous [blocks, block, kv_heads, "
                         "head_dim] caches")
    num_blocks, block_size, heads, head_dim = cache.shape
    out = cache.new_empty((sequence_length, heads, head_dim))
    if sequence_length == 0:
        return out
    code = DTYPE_CODES.get(cache.dtype)
    if code is None:
        dtype_code(cache.dtype)  # raises with the supported dtypes
    status = _lib.load_library().nkv_gather(
        cache.data_ptr(), block_table.data_ptr(), block_table.shape[0], sequence_length,
        block_size, heads * head_dim, num_blocks, code, out.data_ptr(),
        stream_of(cache.get_device()),
    )
    if status:
        _lib.check(status, "nanovllm_paged_kv::gather")
    return out


def _store_impl(key, value, key_cache, value_cache, slot_mapping) -> None:
    _require_device("paged KV HIP Store", key, value, key_cache, value_cache, slot_mapping)
    _require_contiguous_cache("paged KV HIP Store", key_cache, value_cache)
    if key.dtype != value.dtype or key.dtype != key_cache.dtype or key.dtype != value_cache.dtype:
        raise RuntimeError("Paged KV HIP Store dtype mismatch")
    slot_mapping = _int32_index("Paged KV HIP Store", "slot_mapping", slot_mapping)
    _require_store_rows(key, value, key_cache, value_cache, slot_mapping)
    store_checked(key, value, key_cache, value_cache, slot_mapping)


def _gather_impl(cache, block_table, sequence_length: int) -> torch.Tensor:
    _require_device("paged KV HIP Gather", cache, block_table)
    _require_contiguous_cache("paged KV HIP Gather", cache)
    block_table = _int32_index("Paged KV HIP Gather", "block_table", block_table)
    if cache.ndim != 4 or block_table.ndim != 1:
        raise RuntimeError("Paged KV HIP Gather: cache must be [blocks, block, kv_heads, head_dim] "
                           "and block_table one-dimensional")
    return gather_checked(cache, block_table, sequence_length)


def _build_plan_impl(
    block_tables, cu_seqlens_k, total_tokens: int, num_blocks: int, block_size: int,
    row_elems: int, dtype: torch.dtype,
) -> torch.Tensor:
    device = _require_device("paged KV HIP plan", block_tables, cu_seqlens_k)
    cu_seqlens_k = _int32_index("Paged KV HIP plan", "cu_seqlens_k", cu_seqlens_k)
    if block_tables.dtype != torch.int32:
        raise RuntimeError(f"Paged KV HIP plan: block_tables must be int32, got {block_tables.dtype}")
    if block_tables.ndim == 2 and block_tables.stride(1) != 1:
        block_tables = block_tables.contiguous()  # the kernel walks a row through stride(0) only
    num_seqs = cu_seqlens_k.numel() - 1
    code = dtype_code(dtype)
    capacity = _plan_capacity(total_tokens, num_seqs, block_size, row_elems, code)
    plan = torch.empty((capacity, 4), dtype=torch.int32, device=device)
    if capacity == 0:
        return plan
    status = _lib.load_library().nkv_build_gather_plan(
        block_tables.data_ptr(),
        block_tables.stride(0) if block_tables.ndim == 2 else 0,
        cu_seqlens_k.data_ptr(),
        num_seqs,
        total_tokens,
        block_size,
        row_elems,
        num_blocks,
        code,
        plan.data_ptr(),
        capacity,
        _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::build_gather_plan")
    return plan


def _gather_planned_impl(key_cache, value_cache, plan, key_out, value_out) -> None:
    device = _require_device(
        "paged KV HIP varlen Gather", key_cache, value_cache, plan, key_out, value_out
    )
    _require_contiguous_cache("paged KV HIP varlen Gather", key_cache, value_cache)
    if plan.dtype != torch.int32 or plan.ndim != 2 or plan.shape[1] != 4 or not plan.is_contiguous():
        raise ValueError("gather plan must be a contiguous [capacity, 4] int32 tensor")
    if not (key_out.is_contiguous() and value_out.is_contiguous()):
        raise ValueError("varlen Gather outputs must be contiguous")
    if key_out.shape != value_out.shape or key_out.shape[1:] != key_cache.shape[2:]:
        raise ValueError("varlen Gather outputs must be [rows, kv_heads, head_dim] of the caches")
    if key_out.dtype != key_cache.dtype or value_out.dtype != key_cache.dtype:
        raise ValueError("varlen Gather outputs must have the caches' dtype")
    row_elems = key_cache.shape[2] * key_cache.shape[3]
    status = _lib.load_library().nkv_gather_varlen_planned(
        key_cache.data_ptr(),
        value_cache.data_ptr(),
        plan.data_ptr(),
        plan.shape[0],
        key_cache.shape[0] * key_cache.shape[1],
        key_out.shape[0],
        key_cache.shape[1],
        row_elems,
        dtype_code(key_cache.dtype),
        key_out.data_ptr(),
        value_out.data_ptr(),
        _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::gather_varlen_planned")


def _gather_varlen_impl(key_cache, value_cache, block_tables, cu_seqlens_k, total_tokens: int):
    _require_device("paged KV HIP varlen Gather", key_cache, value_cache, block_tables, cu_seqlens_k)
    num_blocks, block_size, heads, head_dim = key_cache.shape
    key_out = torch.empty((total_tokens, heads, head_dim), dtype=key_cache.dtype, device=key_cache.device)
    value_out = torch.empty_like(key_out)
    if total_tokens == 0:
        return key_out, value_out
    plan = _build_plan_impl(
        block_tables, cu_seqlens_k, total_tokens, num_blocks, block_size, heads * head_dim,
        key_cache.dtype,
    )
    _gather_planned_impl(key_cache, value_cache, plan, key_out, value_out)
    return key_out, value_out


def _store_gather_plan_bytes(num_tokens: int, total_tokens: int, num_seqs: int, block_size: int,
                             row_elems: int, code: int) -> int:
    """Bytes of a store+gather plan for these counts (the int32 plan tensor
    holds at least 16 bytes, exactly this many when it is non-zero)."""
    return int(_lib.load_library().nkv_store_gather_plan_bytes(
        num_tokens, total_tokens, num_seqs, block_size, row_elems, code))


def _build_store_gather_plan_impl(
    block_tables, cu_seqlens_q, cu_seqlens_k, num_tokens: int, total_tokens: int,
    num_blocks: int, block_size: int, row_elems: int, dtype: torch.dtype,
) -> torch.Tensor:
    device = _require_device("paged KV HIP store+gather plan", block_tables, cu_seqlens_q,
                             cu_seqlens_k)
    num_seqs = _require_cu("cu_seqlens_q", cu_seqlens_q)
    _require_cu("cu_seqlens_k", cu_seqlens_k, num_seqs)
    if block_tables.dtype != torch.int32 or block_tables.ndim != 2 or not block_tables.is_contiguous():
        raise ValueError("block_tables must be a contiguous two-dimensional int32 tensor")
    code = dtype_code(dtype)
    nbytes = _store_gather_plan_bytes(num_tokens, total_tokens, num_seqs, block_size, row_elems,
                                      code)
    plan = torch.empty(max(nbytes, 16) // 4, dtype=torch.int32, device=device)
    status = _lib.load_library().nkv_build_store_gather_plan(
        block_tables.data_ptr(), block_tables.shape[1], cu_seqlens_q.data_ptr(),
        cu_seqlens_k.data_ptr(), num_seqs, num_tokens, total_tokens, block_size, row_elems,
        num_blocks, code, plan.data_ptr(), nbytes, _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::build_store_gather_plan")
    return plan


def _store_gather_impl(key, value, key_cache, value_cache, slot_mapping, plan, num_seqs: int,
                       key_out, value_out) -> None:
    device = _require_device("paged KV HIP store+gather", key, value, key_cache, value_cache,
                             slot_mapping, plan, key_out, value_out)
    _require_contiguous_cache("paged KV HIP store+gather", key_cache, value_cache)
    if len({t.dtype for t in (key, value, key_cache, value_cache, key_out, value_out)}) != 1:
        raise RuntimeError("Paged KV HIP store+gather dtype mismatch")
    if not (key_out.is_contiguous() and value_out.is_contiguous()):
        raise ValueError("store+gather outputs must be contiguous")
    if key_out.shape != value_out.shape or key_out.shape[1:] != key_cache.shape[2:]:
        raise ValueError("store+gather outputs must be [rows, kv_heads, head_dim] of the caches")
    slot_mapping = _int32_index("Paged KV HIP store+gather", "slot_mapping", slot_mapping)
    _require_store_rows(key, value, key_cache, value_cache, slot_mapping)
    if plan.dtype != torch.int32 or plan.ndim != 1 or not plan.is_contiguous():
        raise ValueError("store+gather plan must be a contiguous 1-D int32 tensor")
    if num_seqs < 0:
        raise ValueError("num_seqs must be non-negative")
    if key.shape[1] > 1 and key.stride(1) != key.shape[2]:
        key = key.contiguous()
    if value.shape[1] > 1 and value.stride(1) != value.shape[2]:
        value = value.contiguous()
    num_blocks, block_size, heads, head_dim = key_cache.shape
    code = dtype_code(key.dtype)
    need = _store_gather_plan_bytes(key.shape[0], key_out.shape[0], num_seqs, block_size,
                                    heads * head_dim, code)
    if plan.numel() * 4 != max(need, 16):
        raise ValueError(f"store+gather plan holds {plan.numel() * 4} bytes, {key.shape[0]} new "
                         f"tokens and {key_out.shape[0]} context rows of {num_seqs} requests "
                         f"need {max(need, 16)}: build it for the same counts")
    status = _lib.load_library().nkv_store_gather(
        key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(),
        slot_mapping.data_ptr(), key.shape[0], key.stride(0), value.stride(0), plan.data_ptr(),
        need, num_seqs, key_out.shape[0], block_size, heads * head_dim, num_blocks, code,
        key_out.data_ptr(), value_out.data_ptr(), _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::store_gather")


def _build_attention_plan_impl(cu_seqlens_k, total_tokens: int, block_size: int,
                               num_kv_heads: int):
    device = _require_device("paged KV HIP attention plan", cu_seqlens_k)
    if cu_seqlens_k.dtype != torch.int32 or cu_seqlens_k.ndim != 1 or not cu_seqlens_k.is_contiguous():
        raise ValueError("cu_seqlens_k must be a contiguous 1-D int32 tensor")
    num_seqs = cu_seqlens_k.numel() - 1
    library = _lib.load_library()
    capacity = int(library.nkv_attention_plan_capacity(total_tokens, num_seqs, block_size))
    plan = torch.empty((capacity, 4), dtype=torch.int32, device=device)
    first_part = torch.empty(num_seqs + 1, dtype=torch.int32, device=device)
    status = library.nkv_build_attention_plan(
        cu_seqlens_k.data_ptr(),
        num_seqs,
        block_size,
        num_kv_heads,
        plan.data_ptr() if capacity else None,
        capacity,
        first_part.data_ptr(),
        _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::build_attention_plan")
    return plan, first_part


def _paged_attention_decode_impl(q, key_cache, value_cache, block_tables, plan, first_part,
                                 scale: float, out) -> None:
    device = _require_device(
        "paged KV HIP attention", q, key_cache, value_cache, block_tables, plan, first_part, out
    )
    if (block_tables.dtype != torch.int32 or block_tables.ndim != 2
            or block_tables.shape[0] != q.shape[0] or not block_tables.is_contiguous()):
        raise ValueError("block_tables must be a contiguous [num_seqs, width] int32 tensor")
    _require_contiguous_cache("paged KV HIP attention", key_cache, value_cache)
    _require_attention_dtype("paged attention decode", q, key_cache, value_cache, out)
    if q.ndim != 3 or q.stride(2) != 1 or q.stride(1) != q.shape[2]:
        raise ValueError("q must be [num_seqs, num_q_heads, head_dim] with contiguous heads")
    if out.shape != q.shape or out.stride(2) != 1 or out.stride(1) != out.shape[2]:
        raise ValueError("out must match q's shape with contiguous heads")
    num_blocks, block_size, num_kv_heads, head_dim = key_cache.shape
    if q.shape[2] != head_dim:
        raise ValueError("q head_dim does not match the cache")
    if plan.dtype != torch.int32 or plan.ndim != 2 or plan.shape[1] != 4 or not plan.is_contiguous():
        raise ValueError("attention plan must be a contiguous [capacity, 4] int32 tensor")
    if first_part.dtype != torch.int32 or first_part.numel() != q.shape[0] + 1:
        raise ValueError("first_part must be int32 with num_seqs + 1 entries")
    library = _lib.load_library()
    capacity = plan.shape[0]
    nbytes = int(library.nkv_attention_workspace_bytes(capacity, q.shape[1], head_dim))
    workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=device)
    status = library.nkv_paged_attention_decode(
        q.data_ptr(), q.stride(0), key_cache.data_ptr(), value_cache.data_ptr(),
        block_tables.data_ptr(), block_tables.shape[1],
        plan.data_ptr() if capacity else None, capacity, first_part.data_ptr(), q.shape[0],
        num_kv_heads, q.shape[1], head_dim, block_size, num_blocks, float(scale),
        DTYPE_CODES[q.dtype], workspace.data_ptr(), workspace.numel(), out.data_ptr(),
        out.stride(0), _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::paged_attention_decode")


def _require_attention_dtype(what: str, q, key_cache, value_cache, out) -> None:
    """The attention kernels compute in bf16 or fp16 (fp32 accumulation); q,
    the caches and the output share that type."""
    if q.dtype not in (torch.bfloat16, torch.float16) or any(
            t.dtype != q.dtype for t in (key_cache, value_cache, out)):
        raise ValueError(f"{what} supports bfloat16 or float16 q, caches and output of one dtype")


def _require_cu(name: str, cu: torch.Tensor, num_seqs: int | None = None) -> int:
    if cu.dtype != torch.int32 or cu.ndim != 1 or not cu.is_contiguous() or cu.numel() < 1:
        raise ValueError(f"{name} must be a contiguous 1-D int32 tensor of num_seqs + 1 entries")
    if num_seqs is not None and cu.numel() != num_seqs + 1:
        raise ValueError(f"{name} must have num_seqs + 1 entries")
    return cu.numel() - 1


def _build_prefill_plan_impl(cu_seqlens_q, cu_seqlens_k, total_q_tokens: int, group: int):
    device = _require_device("paged KV HIP prefill plan", cu_seqlens_q, cu_seqlens_k)
    num_seqs = _require_cu("cu_seqlens_q", cu_seqlens_q)
    _require_cu("cu_seqlens_k", cu_seqlens_k, num_seqs)
    library = _lib.load_library()
    capacity = int(library.nkv_prefill_plan_capacity(total_q_tokens, num_seqs, group))
    if capacity == 0 and total_q_tokens > 0:
        raise ValueError("prefill attention supports 1 to 8 query heads per kv head")
    plan = torch.empty((capacity, 4), dtype=torch.int32, device=device)
    status = library.nkv_build_prefill_plan(
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), num_seqs, group,
        plan.data_ptr() if capacity else None, capacity, _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::build_prefill_plan")
    return plan


def _paged_attention_prefill_impl(q, key_cache, value_cache, block_tables, cu_seqlens_q,
                                  cu_seqlens_k, plan, scale: float, out) -> None:
    device = _require_device("paged KV HIP prefill attention", q, key_cache, value_cache,
                             block_tables, cu_seqlens_q, cu_seqlens_k, plan, out)
    num_seqs = _require_cu("cu_seqlens_q", cu_seqlens_q)
    _require_cu("cu_seqlens_k", cu_seqlens_k, num_seqs)
    if (block_tables.dtype != torch.int32 or block_tables.ndim != 2
            or block_tables.shape[0] != num_seqs or not block_tables.is_contiguous()):
        raise ValueError("block_tables must be a contiguous [num_seqs, width] int32 tensor")
    _require_contiguous_cache("paged KV HIP prefill attention", key_cache, value_cache)
    _require_attention_dtype("paged attention prefill", q, key_cache, value_cache, out)
    if q.ndim != 3 or q.stride(2) != 1 or q.stride(1) != q.shape[2]:
        raise ValueError("q must be [tokens, num_q_heads, head_dim] with contiguous heads")
    if out.shape != q.shape or out.stride(2) != 1 or out.stride(1) != out.shape[2]:
        raise ValueError("out must match q's shape with contiguous heads")
    num_blocks, block_size, num_kv_heads, head_dim = key_cache.shape
    if q.shape[2] != head_dim:
        raise ValueError("q head_dim does not match the cache")
    if plan.dtype != torch.int32 or plan.ndim != 2 or plan.shape[1] != 4 or not plan.is_contiguous():
        raise ValueError("prefill plan must be a contiguous [capacity, 4] int32 tensor")
    library = _lib.load_library()
    if num_kv_heads > 0 and q.shape[1] % num_kv_heads == 0:
        # A plan built for these queries and this head layout has at least
        # this many entries; one built for a layout with longer query tiles
        # has fewer (its tiles would not fit this kernel's).
        need = int(library.nkv_prefill_plan_capacity(q.shape[0], num_seqs,
                                                     q.shape[1] // num_kv_heads))
        if plan.shape[0] < need:
            raise ValueError(f"prefill plan has {plan.shape[0]} entries, these queries need {need}: "
                             "build it with build_prefill_plan for the same q and cu_seqlens")
    status = library.nkv_paged_attention_prefill(
        q.data_ptr(), q.stride(0), key_cache.data_ptr(), value_cache.data_ptr(),
        block_tables.data_ptr(), block_tables.shape[1], cu_seqlens_q.data_ptr(),
        cu_seqlens_k.data_ptr(), plan.data_ptr() if plan.shape[0] else None, plan.shape[0],
        num_seqs, num_kv_heads, q.shape[1], head_dim, block_size, num_blocks, float(scale),
        DTYPE_CODES[q.dtype], out.data_ptr(), out.stride(0), _stream(device),
    )
    _lib.check(status, "nanovllm_paged_kv::paged_attention_prefill")


def register_ops() -> None:
    """Define the schemas (unless another library already did) and register
    the HIP implementations on the CUDA key.  Idempotent."""
    global _FRAGMENT
    with _REGISTER_LOCK:
        if _FRAGMENT is not None:
            return
        fragment = torch.library.Library(NAMESPACE, "FRAGMENT")
        namespace = getattr(torch.ops, NAMESPACE)
        for name, schema in SCHEMAS.items():
            if not hasattr(namespace, name):
                fragment.define(schema)
        fragment.impl("store", _store_impl, "CUDA")
        fragment.impl("gather", _gather_impl, "CUDA")
        fragment.impl("gather_varlen", _gather_varlen_impl, "CUDA")
        fragment.impl("build_gather_plan", _build_plan_impl, "CUDA")
        fragment.impl("gather_varlen_planned", _gather_planned_impl, "CUDA")
        fragment.impl("build_attention_plan", _build_attention_plan_impl, "CUDA")
        fragment.impl("paged_attention_decode", _paged_attention_decode_impl, "CUDA")
        fragment.impl("build_store_gather_plan", _build_store_gather_plan_impl, "CUDA")
        fragment.impl("store_gather", _store_gather_impl, "CUDA")
        fragment.impl("build_prefill_plan", _build_prefill_plan_impl, "CUDA")
        fragment.impl("paged_attention_prefill", _paged_attention_prefill_impl, "CUDA")
        _FRAGMENT = fragment


# The backend object calls the implementations directly: the registered ops
# dispatch to these same functions, and skipping the dispatcher hop saves
# ~1.4 us of host time per call.
store = _store_impl
gather = _gather_impl
gather_varlen = _gather_varlen_impl
build_gather_plan = _build_plan_impl
gather_varlen_planned = _gather_planned_impl
build_attention_plan = _build_attention_plan_impl
paged_attention_decode = _paged_attention_decode_impl
build_prefill_plan = _build_prefill_plan_impl
paged_attention_prefill = _paged_attention_prefill_impl
build_store_gather_plan = _build_store_gather_plan_impl
store_gather = _store_gather_impl
