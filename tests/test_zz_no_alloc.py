"""nkv_gather_varlen_noalloc (the varlen gather whose plan lives in the
library's own device array) against nkv_gather_varlen (the same gather with
a caller workspace), bit-exact, through the C ABI.

Two calls in a row share the one array of the GPU: the second, smaller call
must not see anything the first left behind.  A plan that fills the array
exactly is accepted, and one row more is rejected before any device work.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from nanokv import _lib
from oracle import paged_kv as oracle

pytestmark = pytest.mark.gpu

SENTINEL = 0x7BCD


def _case(rng, num_seqs, max_len, block_size, heads, dim, dtype, device, spare_blocks=5):
    lens = rng.integers(0, max_len + 1, num_seqs)
    lens[rng.integers(0, num_seqs)] = max_len
    need = -(-lens // block_size)
    nb = int(need.sum()) + spare_blocks
    perm = rng.permutation(nb).astype(np.int32)
    width = int(need.max()) + 1
    tables = np.full((num_seqs, width), -1, np.int32)
    cursor = 0
    for i, n in enumerate(need.tolist()):
        tables[i, :n] = perm[cursor:cursor + n]
        cursor += n
    gen = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    shape = (nb, block_size, heads, dim)
    kc = torch.randn(shape, generator=gen).to(dtype)
    vc = torch.randn(shape, generator=gen).to(dtype)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    return {
        "lens": lens, "tables": tables, "cu": cu, "host_k": kc, "host_v": vc,
        "kc": kc.to(device), "vc": vc.to(device),
        "d_tables": torch.from_numpy(tables).to(device), "d_cu": torch.from_numpy(cu).to(device),
        "total": int(cu[-1]), "block_size": block_size, "row_elems": heads * dim,
        "num_blocks": nb, "dtype": dtype,
    }


def _dtype_code(dtype):
    return {torch.float16: _lib.NKV_DTYPE_FLOAT16, torch.bfloat16: _lib.NKV_DTYPE_BFLOAT16,
            torch.float32: _lib.NKV_DTYPE_FLOAT32}[dtype]


def _outputs(case, device):
    shape = (case["total"],) + tuple(case["kc"].shape[2:])
    k_out = torch.empty(shape, dtype=case["dtype"], device=device)
    k_out.view(torch.int16).fill_(SENTINEL)
    return k_out, k_out.clone()


def _run(lib, case, device, *, noalloc: bool):
    k_out, v_out = _outputs(case, device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
    num_seqs = case["d_tables"].shape[0]
    args = (case["kc"].data_ptr(), case["vc"].data_ptr(), case["d_tables"].data_ptr(),
            case["d_tables"].shape[1], case["d_cu"].data_ptr(), num_seqs, case["total"],
            case["block_size"], case["row_elems"], case["num_blocks"], _dtype_code(case["dtype"]),
            k_out.data_ptr(), v_out.data_ptr())
    if noalloc:
        _lib.check(lib.nkv_gather_varlen_noalloc(*args, stream), "nkv_gather_varlen_noalloc")
        return k_out, v_out
    capacity = lib.nkv_gather_plan_capacity(case["total"], num_seqs, case["block_size"],
                                            case["row_elems"], _dtype_code(case["dtype"]))
    workspace = torch.empty(16 * capacity, dtype=torch.uint8, device=device)
    _lib.check(lib.nkv_gather_varlen(*args, workspace.data_ptr(), workspace.numel(), stream),
               "nkv_gather_varlen")
    torch.cuda.synchronize(device)
    return k_out, v_out


def _words(t):
    return t.cpu().view(torch.int16).numpy()


def _check(lib, case, device):
    expect_k, expect_v = _run(lib, case, device, noalloc=False)
    got_k, got_v = _run(lib, case, device, noalloc=True)
    torch.cuda.synchronize(device)
    np.testing.assert_array_equal(_words(got_k), _words(expect_k))
    np.testing.assert_array_equal(_words(got_v), _words(expect_v))
    # and both are the concatenated per-request gathers of the oracle
    np.testing.assert_array_equal(
        _words(got_k), oracle.gather_varlen(case["host_k"].view(torch.int16).numpy(),
                                            case["tables"], case["lens"]))


def test_noalloc_matches_workspace_entry_point_two_calls(gpu_device):
    lib = _lib.load_library()
    rng = np.random.default_rng(20260)
    first = _case(rng, 211, 3000, 256, 8, 128, torch.bfloat16, gpu_device)
    print(f"[no-alloc] call 1: {first['total']} rows, 211 seqs, 8x128 bf16", flush=True)
    _check(lib, first, gpu_device)
    second = _case(rng, 9, 700, 16, 2, 128, torch.float16, gpu_device)
    assert second["total"] < first["total"]
    print(f"[no-alloc] call 2: {second['total']} rows, 9 seqs, 2x128 f16", flush=True)
    _check(lib, second, gpu_device)


def test_noalloc_plan_that_fills_the_scratch(gpu_device):
    """Block size 1 makes one plan entry per row: total_rows + num_seqs
    entries of 16 bytes fill the array exactly; one row more is rejected
    with NKV_E_CAPACITY and the outputs stay untouched."""
    lib = _lib.load_library()
    entries = _lib.NKV_SCRATCH_BYTES // 16
    num_seqs = 64
    rng = np.random.default_rng(7)
    lens = np.full(num_seqs, (entries - num_seqs) // num_seqs, np.int64)
    lens[-1] += (entries - num_seqs) - int(lens.sum())
    perm = rng.permutation(int(lens.sum()) + 3).astype(np.int32)
    tables = np.full((num_seqs, int(lens.max())), -1, np.int32)
    cursor = 0
    for i, n in enumerate(lens.tolist()):
        tables[i, :n] = perm[cursor:cursor + n]
        cursor += n
    gen = torch.Generator().manual_seed(3)
    nb = perm.size
    host_k = torch.randn((nb, 1, 1, 64), generator=gen).to(torch.float16)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    case = {"lens": lens, "tables": tables, "cu": cu, "host_k": host_k, "host_v": host_k,
            "kc": host_k.to(gpu_device), "vc": (host_k + 1).to(gpu_device),
            "d_tables": torch.from_numpy(tables).to(gpu_device),
            "d_cu": torch.from_numpy(cu).to(gpu_device), "total": int(cu[-1]), "block_size": 1,
            "row_elems": 64, "num_blocks": nb, "dtype": torch.float16}
    capacity = lib.nkv_gather_plan_capacity(case["total"], num_seqs, 1, 64, _lib.NKV_DTYPE_FLOAT16)
    assert capacity == entries
    print(f"[no-alloc] full scratch: {case['total']} rows, {capacity} plan entries", flush=True)
    _check(lib, case, gpu_device)

    k_out, v_out = _outputs(case, gpu_device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu_device).cuda_stream)
    status = lib.nkv_gather_varlen_noalloc(
        case["kc"].data_ptr(), case["vc"].data_ptr(), case["d_tables"].data_ptr(),
        tables.shape[1], case["d_cu"].data_ptr(), num_seqs, case["total"] + 1, 1, 64, nb,
        _lib.NKV_DTYPE_FLOAT16, k_out.data_ptr(), v_out.data_ptr(), stream)
    assert status == 3  # NKV_E_CAPACITY
    assert b"scratch" in lib.nkv_last_error()
    torch.cuda.synchronize(gpu_device)
    assert (k_out.view(torch.int16) == SENTINEL).all()


def test_noalloc_allocates_nothing_on_later_calls(gpu_device):
    """After a first call (which loads the kernels and the array with the
    library's code object), calls change neither the device's free memory
    nor torch's allocations."""
    lib = _lib.load_library()
    rng = np.random.default_rng(99)
    case = _case(rng, 37, 2000, 256, 8, 128, torch.bfloat16, gpu_device)
    k_out, v_out = _outputs(case, gpu_device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu_device).cuda_stream)
    args = (case["kc"].data_ptr(), case["vc"].data_ptr(), case["d_tables"].data_ptr(),
            case["d_tables"].shape[1], case["d_cu"].data_ptr(), 37, case["total"],
            256, 1024, case["num_blocks"], _lib.NKV_DTYPE_BFLOAT16, k_out.data_ptr(),
            v_out.data_ptr(), stream)
    _lib.check(lib.nkv_gather_varlen_noalloc(*args), "nkv_gather_varlen_noalloc")
    torch.cuda.synchronize(gpu_device)
    free_before, _ = torch.cuda.mem_get_info(gpu_device)
    allocated_before = torch.cuda.memory_allocated(gpu_device)
    for _ in range(5):
        _lib.check(lib.nkv_gather_varlen_noalloc(*args), "nkv_gather_varlen_noalloc")
    torch.cuda.synchronize(gpu_device)
    assert torch.cuda.mem_get_info(gpu_device)[0] == free_before
    assert torch.cuda.memory_allocated(gpu_device) == allocated_before


# Run in a fresh interpreter, so that the entry point's first call on the
# device (its one-time scratch address lookup) happens inside the capture.
GRAPH_CHILD = r'''
import ctypes, sys
import numpy as np
import torch
sys.path[:0] = [sys.argv[1], sys.argv[2]]
from nanokv import _lib
lib = _lib.load_library()
dev = torch.device("cuda", 0)
rng = np.random.default_rng(5)
bs, heads, dim, seqs = 16, 2, 128, 23
lens = rng.integers(0, 400, seqs)
need = -(-lens // bs)
nb = int(need.sum()) + 4
perm = rng.permutation(nb).astype(np.int32)
tables = np.full((seqs, int(need.max()) + 1), -1, np.int32)
c = 0
for i, n in enumerate(need.tolist()):
    tables[i, :n] = perm[c:c + n]
    c += n
cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
total = int(cu[-1])
kc = torch.randn(nb, bs, heads, dim, device=dev).to(torch.bfloat16)
vc = torch.randn_like(kc)
d_tables, d_cu = torch.from_numpy(tables).to(dev), torch.from_numpy(cu).to(dev)
k_out = torch.empty(total, heads, dim, dtype=torch.bfloat16, device=dev)
v_out = torch.empty_like(k_out)
cap = lib.nkv_gather_plan_capacity(total, seqs, bs, heads * dim, _lib.NKV_DTYPE_BFLOAT16)
workspace = torch.empty(16 * cap, dtype=torch.uint8, device=dev)

def call(entry, stream, ko, vo, *extra):
    args = (kc.data_ptr(), vc.data_ptr(), d_tables.data_ptr(), tables.shape[1], d_cu.data_ptr(),
            seqs, total, bs, heads * dim, nb, _lib.NKV_DTYPE_BFLOAT16, ko.data_ptr(), vo.data_ptr())
    _lib.check(entry(*args, *extra, ctypes.c_void_p(stream)), "call")

torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
with torch.cuda.graph(graph, stream=side):
    call(lib.nkv_gather_varlen_noalloc, side.cuda_stream, k_out, v_out)
expect_k, expect_v = torch.empty_like(k_out), torch.empty_like(v_out)
for replay in range(4):
    kc.copy_(torch.randn(kc.shape, device=dev).to(torch.bfloat16))   # eager work between replays
    vc.copy_(torch.randn(vc.shape, device=dev).to(torch.bfloat16))
    k_out.fill_(0)
    v_out.fill_(0)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    call(lib.nkv_gather_varlen, torch.cuda.current_stream().cuda_stream, expect_k, expect_v,
         workspace.data_ptr(), workspace.numel())
    torch.cuda.synchronize()
    same = (torch.equal(k_out.view(torch.int16), expect_k.view(torch.int16))
            and torch.equal(v_out.view(torch.int16), expect_v.view(torch.int16)))
    print(f"replay {replay}: {'equal' if same else 'DIFFERENT'} ({total} rows)", flush=True)
    if not same:
        sys.exit(1)
print("graph ok", flush=True)
'''


def test_noalloc_first_call_under_graph_capture(gpu_device):
    """A fresh process whose first call of the entry point is made while a
    graph is being captured; the graph is replayed four times, with eager
    work and synchronisations between the replays, each replay bit-exact
    against the workspace entry point on the same (changed) caches."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    print("[no-alloc] graph capture in a fresh process", flush=True)
    done = subprocess.run([sys.executable, "-c", GRAPH_CHILD, str(root),
                           str(root / "nano-vllm-multimodal_amd")],
                          capture_output=True, text=True, timeout=180)
    print(done.stdout[-2000:], done.stderr[-2000:], flush=True)
    assert done.returncode == 0
    assert done.stdout.count("equal") == 4 and "graph ok" in done.stdout
