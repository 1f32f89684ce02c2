"""The hip backend's native cache owner and async slot upload, mirroring
the reference's runtime-owner tests (tests/test_paged_kv_cuda.py:155-273):
native allocation, pinned async copy on a side stream, empty input, grown
buffer reuse, retention of an ephemeral host tensor, and a 64-step decode
replay where every step's slot goes up through the transfer lane."""
from __future__ import annotations

import gc

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture()
def backend(gpu_device):
    from nanokv.paged_kv import create_paged_kv_backend

    return create_paged_kv_backend("hip")


def test_allocation_has_native_owner(backend):
    allocation = backend.allocate((2, 5, 8, 2, 128), dtype=torch.bfloat16, device="cuda")
    assert allocation.owner is not None
    assert allocation.tensor.shape == (2, 5, 8, 2, 128)
    assert allocation.tensor.data_ptr() == allocation.owner.tensor().data_ptr()
    assert allocation.owner.pending_host_copy_count() == 0


def test_async_copies_pinned_slot_mapping_on_side_stream(backend):
    allocation = backend.allocate((2, 1, 8, 1, 64), dtype=torch.float16, device="cuda")
    host_slots = torch.tensor([0, 3, 7], dtype=torch.int32).pin_memory()
    with torch.cuda.stream(torch.cuda.Stream()):
        device_slots = backend.copy_slots_async(allocation, host_slots)
        torch.cuda.current_stream().synchronize()
    assert device_slots.device.type == "cuda"
    assert torch.equal(device_slots.cpu(), host_slots)


def test_async_copy_accepts_empty_slot_mapping(backend):
    allocation = backend.allocate((2, 1, 8, 1, 64), dtype=torch.float16, device="cuda")
    device_slots = backend.copy_slots_async(allocation, torch.empty(0, dtype=torch.int32, pin_memory=True))
    assert device_slots.device.type == "cuda"
    assert device_slots.dtype == torch.int32
    assert device_slots.numel() == 0


def test_async_copy_reuses_grown_slot_buffer(backend):
    allocation = backend.allocate((2, 1, 8, 1, 64), dtype=torch.float16, device="cuda")
    first = backend.copy_slots_async(allocation, torch.tensor([0, 3, 7, 2], dtype=torch.int32).pin_memory())
    torch.cuda.current_stream().synchronize()
    second_host = torch.tensor([6, 1], dtype=torch.int32).pin_memory()
    second = backend.copy_slots_async(allocation, second_host)
    torch.cuda.current_stream().synchronize()
    assert first.data_ptr() == second.data_ptr()
    assert torch.equal(second.cpu(), second_host)
    grown_host = torch.arange(9, dtype=torch.int32).pin_memory()
    grown = backend.copy_slots_async(allocation, grown_host)
    torch.cuda.current_stream().synchronize()
    assert torch.equal(grown.cpu(), grown_host)


def test_async_copy_retains_ephemeral_pinned_host_tensor(backend):
    allocation = backend.allocate((2, 1, 8, 1, 64), dtype=torch.float16, device="cuda")
    host_slots = torch.tensor([0, 3, 7], dtype=torch.int32).pin_memory()
    device_slots = backend.copy_slots_async(allocation, host_slots)
    assert allocation.owner.pending_host_copy_count() == 1
    del host_slots
    gc.collect()
    torch.cuda.current_stream().synchronize()
    assert device_slots.tolist() == [0, 3, 7]
    # Completed copies are released at the next upload (paged_kv.cpp:110,156-167).
    backend.copy_slots_async(allocation, torch.tensor([1], dtype=torch.int32).pin_memory())
    assert allocation.owner.pending_host_copy_count() <= 1


def test_repeated_async_slot_copy_and_store_matches_decode_sequence(backend):
    allocation = backend.allocate((2, 1, 16, 1, 64), dtype=torch.float16, device="cuda")
    allocation.tensor.fill_(-1)
    key_cache, value_cache = allocation.tensor[0], allocation.tensor[1]
    for step in range(64):
        key = torch.full((1, 1, 64), step, dtype=torch.float16, device="cuda")
        host_slot = torch.tensor([step % 16], dtype=torch.int32, pin_memory=True)
        device_slot = backend.copy_slots_async(allocation, host_slot)
        del host_slot
        backend.store(key, -key, key_cache, value_cache, device_slot)
    torch.cuda.synchronize()
    expected = torch.arange(48, 64, dtype=torch.float16, device="cuda")
    assert torch.equal(key_cache[0, :, 0, 0], expected), key_cache[0, :, 0, 0].tolist()
    assert torch.equal(value_cache[0, :, 0, 0], -expected)


@pytest.mark.parametrize("make,message", [
    (lambda: torch.tensor([1, 2], dtype=torch.int32, device="cuda"), "CPU tensor"),
    (lambda: torch.tensor([1, 2], dtype=torch.int64).pin_memory(), "int32"),
    (lambda: torch.zeros((2, 2), dtype=torch.int32).pin_memory(), "one-dimensional"),
    (lambda: torch.tensor([1, 2], dtype=torch.int32), "pinned"),
])
def test_async_copy_rejects_bad_sources(backend, make, message):
    allocation = backend.allocate((2, 1, 8, 1, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError, match=message):
        backend.copy_slots_async(allocation, make())
