"""CPU tests of the C ABI library: it is built for gfx950, loads without a
GPU, exports every function include/nanokv.h declares, and rejects
host-visible contract violations before any device work (these calls never
reach the HIP runtime)."""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

from nanokv import _lib
from nanokv.build import LIBRARY_PATH

HEADER = Path(__file__).resolve().parents[1] / "include" / "nanokv.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(nkv_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_agree():
    declared = declared_functions()
    assert declared, "no declarations parsed"
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    assert LIBRARY_PATH.is_file(), "run __graft_entry__.build() first"
    library = _lib.load_library()
    declared = declared_functions()
    for name in declared:
        assert hasattr(library, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(LIBRARY_PATH)], capture_output=True, text=True)
    exported = set(re.findall(r"\bT (nkv_[a-z0-9_]+)\b", nm.stdout))
    assert declared <= exported, declared - exported


def test_library_carries_gfx950_code_object():
    data = LIBRARY_PATH.read_bytes()
    assert b"gfx950" in data


def test_version_and_plan_geometry():
    lib = _lib.load_library()
    assert lib.nkv_version() >= 100
    # chunk rows divide the block size and never exceed it
    for block_size, row_elems, dtype in ((256, 1024, 1), (256, 256, 1), (16, 80, 2), (16, 15, 0), (4, 5, 0)):
        rows = lib.nkv_gather_plan_rows(block_size, row_elems, dtype)
        assert 1 <= rows <= block_size and block_size % rows == 0
    assert lib.nkv_gather_plan_rows(256, 1024, 1) == 16  # 32 KiB chunks of 2 KiB rows
    assert lib.nkv_gather_plan_rows(0, 1024, 1) == 0
    assert lib.nkv_gather_plan_rows(256, 1024, 7) == 0
    assert lib.nkv_gather_plan_capacity(1000, 4, 256, 1024, 1) == -(-1000 // 16) + 4
    assert lib.nkv_gather_plan_capacity(0, 0, 256, 1024, 1) == 0
    # store+gather plan: 8 bytes per token (rounded to 16) + 16 per chunk of cached rows
    cap = lib.nkv_gather_plan_capacity(1000, 4, 256, 1024, 1)
    assert lib.nkv_store_gather_plan_bytes(5, 1000, 4, 256, 1024, 1) == 48 + 16 * cap
    assert lib.nkv_store_gather_plan_bytes(0, 0, 0, 256, 1024, 1) == 0
    # the plan of the rejection cases below: 8 tokens, 40 rows of 16 bytes in
    # chunks of 16 rows, 2 requests -> 64 + 16 * (3 + 2)
    assert lib.nkv_store_gather_plan_bytes(8, 40, 2, 16, 8, 1) == 144


@pytest.mark.parametrize("call,message", [
    (lambda l: l.nkv_store(None, None, None, None, None, 1, 1, 1, 1, 1, 99, None), "dtype"),
    (lambda l: l.nkv_store(None, None, None, None, None, -1, 1, 1, 1, 1, 1, None), "negative"),
    (lambda l: l.nkv_store(None, None, None, None, None, 4, 8, 8, 8, 64, 1, None), "null"),
    (lambda l: l.nkv_gather(None, None, 1, 5, 4, 8, 3, 1, None, None), "cover"),
    (lambda l: l.nkv_gather(None, None, 2, -1, 4, 8, 3, 1, None, None), "non-negative"),
    (lambda l: l.nkv_gather(None, None, 2, 5, 0, 8, 3, 1, None, None), "positive"),
    (lambda l: l.nkv_build_gather_plan(None, 4, None, 9000, 10, 4, 8, 3, 1, None, 16, None), "num_seqs"),
    (lambda l: l.nkv_gather_varlen_planned(None, None, None, 4, 8, 8, 4, 8, 1, None, None, None), "null"),
    (lambda l: l.nkv_gather_varlen(None, None, None, 1, None, 2, 100, 16, 8, 4, 1, None, None, None, 16, None), "workspace"),
    (lambda l: l.nkv_gather_varlen_noalloc(None, None, None, 1, None, 2, 10**8, 256, 1024, 4, 1, None, None, None), "scratch"),
    (lambda l: l.nkv_gather_varlen_noalloc(None, None, None, 1, None, 2, -1, 256, 1024, 4, 1, None, None, None), "non-negative"),
    (lambda l: l.nkv_paged_attention_decode(None, 2048, None, None, None, 4, None, 4, None, 1, 8, 16, 128,
                                            256, 16, 0.0, 1, None, 0, None, 2048, None), "positive"),
    (lambda l: l.nkv_paged_attention_decode(None, 2048, None, None, None, 4, None, 4, None, 1, 2, 16, 128,
                                            256, 16, -0.5, 1, None, 0, None, 2048, None), "positive"),
    (lambda l: l.nkv_paged_attention_decode(None, 2048, None, None, None, 4, None, 4, None, 1, 8, 16, 128,
                                            256, 16, float("nan"), 1, None, 0, None, 2048, None), "finite"),
    # the range split (fewer than 8 kv heads) needs its whole plan
    (lambda l: l.nkv_paged_attention_decode(None, 2048, None, None, None, 4, None, 4, None, 1, 2, 16, 128,
                                            256, 16, 0.1, 1, None, 0, None, 2048, None), "plan capacity"),
    (lambda l: l.nkv_build_attention_plan(None, 1, 256, 2, None, 4, None, None), "capacity 4"),
    (lambda l: l.nkv_build_attention_plan(None, 1, 256, 0, None, 4096, None, None), "num_kv_heads"),
    (lambda l: l.nkv_build_store_gather_plan(None, 4, None, None, 5000, 8, 40, 16, 8, 10, 1, None, 144,
                                             None), "num_seqs"),
    (lambda l: l.nkv_build_store_gather_plan(None, 4, None, None, 2, 8, 40, 16, 8, 10, 1, None, 16,
                                             None), "plan of 16 bytes"),
    (lambda l: l.nkv_build_store_gather_plan(None, 4, None, None, 2, 8, 40, 16, 8, 10, 1, None, 4096,
                                             None), "exactly 144"),
    (lambda l: l.nkv_build_store_gather_plan(None, -4, None, None, 2, 8, 40, 16, 8, 10, 1, None, 144,
                                             None), "table_stride"),
    (lambda l: l.nkv_build_store_gather_plan(None, 4, None, None, 2, 8, 40, 16, 8, 10, 1, None, 144,
                                             None), "null"),
    (lambda l: l.nkv_store_gather(None, None, None, None, None, 8, 8, 8, None, 16, 2, 40, 16, 8, 10, 1,
                                  None, None, None), "plan of 16 bytes"),
    (lambda l: l.nkv_store_gather(None, None, None, None, None, 8, 8, 8, None, 4096, 2, 40, 16, 8, 10, 1,
                                  None, None, None), "exactly 144"),
    (lambda l: l.nkv_store_gather(None, None, None, None, None, -1, 8, 8, None, 144, 2, 40, 16, 8, 10, 1,
                                  None, None, None), "out of range"),
    (lambda l: l.nkv_store_gather(None, None, None, None, None, 8, 8, 8, None, 144, 2, 40, 16, 8, 10, 1,
                                  None, None, None), "null"),
    (lambda l: l.nkv_pack_decode(None, None, None, 0, 5000, 5000, 16, 4, 4, None, None, None, None, None), "num_seqs"),
    (lambda l: l.nkv_pack_decode(None, None, None, 0, 3, 3, 16, 4, 4, None, None, None, None, None), "null"),
    (lambda l: l.nkv_pack_decode(None, None, None, 0, 3, 2, 16, 4, 4, None, None, None, None, None), "padded_seqs"),
    (lambda l: l.nkv_pack_decode(None, None, None, 0, 3, 3, 16, 4, 2, None, None, None, None, None), "table_stride"),
    (lambda l: l.nkv_pack_prefill(None, None, None, None, None, 0, 3, 0, 4, 8, None, None, None, None, None, None, None, None), "block_size"),
])
def test_contract_violations_fail_before_launch(call, message):
    lib = _lib.load_library()
    status = call(lib)
    assert status != 0
    assert message in lib.nkv_last_error().decode()
    with pytest.raises(RuntimeError, match=message):
        _lib.check(status, "probe")
