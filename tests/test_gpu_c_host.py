"""The library driven from C: tests/c_host/abi_host (built by
__graft_entry__.build() from tests/c_host/abi_host.c) allocates its own
device buffers and stream with the HIP runtime, calls nkv_store, nkv_gather,
nkv_gather_varlen (caller workspace and no-alloc) and one rejected NULL key
through the C ABI with no Python in between, and compares every byte with
the oracle's C restatement."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BINARY = Path(__file__).resolve().parent / "c_host" / "_build" / "abi_host"


def test_c_host_program_matches_the_oracle(gpu_device):
    if not BINARY.is_file():
        pytest.fail(f"{BINARY} is missing: run __graft_entry__.build() first")
    result = subprocess.run([str(BINARY)], capture_output=True, text=True, timeout=120)
    assert result.returncode == 0, f"abi_host exited {result.returncode}:\n{result.stdout}{result.stderr}"
    assert "abi_host ok" in result.stdout
