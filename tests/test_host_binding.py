"""The C++ host binding of the hip backend's per-call store and gather
(csrc/nkv_host.cpp), on the host: its checks restate the reference
validators (nanovllm/layers/paged_kv/base.py:75-151, restated in Python as
nanokv.paged_kv.base.check_store_inputs / check_gather_inputs), so every
input is held to the same outcome in both, the same ValueError message or
none, over the reference's own bad-input cases and more; and the binding
refuses to run before it is bound, and reports its build id."""
from __future__ import annotations

import os
from unittest.mock import patch

import pytest
import torch

from nanokv import _lib
from nanokv import build as nkv_build
from nanokv.paged_kv.base import check_gather_inputs, check_store_inputs


@pytest.fixture(scope="module")
def host():
    return _lib.load_host()


def _outcome(fn, *args):
    try:
        fn(*args)
    except ValueError as exc:
        return str(exc)
    return None


def store_inputs():
    key = torch.arange(3 * 2 * 4, dtype=torch.float32).reshape(3, 2, 4)
    return key, key + 100, torch.full((3, 4, 2, 4), -1.0), torch.full((3, 4, 2, 4), -1.0), \
        torch.tensor([0, 5, -1], dtype=torch.int32)


def store_cases():
    key, value, kc, vc, slots = store_inputs()
    yield "valid", (key, value, kc, vc, slots)
    yield "short key", (key[:2], value, kc, vc, slots)
    yield "2-d key", (key[0], value[0], kc, vc, slots)
    yield "narrow cache", (key, value, kc[:, :, :1], vc, slots)
    yield "cache dims", (key, value, kc[0], vc[0], slots)
    yield "cache head_dim", (key, value, kc[..., :2], vc[..., :2], slots)
    yield "int64 slots", (key, value, kc, vc, slots.to(torch.int64))
    yield "2-d slots", (key, value, kc, vc, slots.view(3, 1))
    yield "transposed", (key.transpose(1, 2), value.transpose(1, 2), kc, vc, slots)
    yield "value dtype", (key, value.to(torch.float16), kc, vc, slots)
    yield "cache dtype", (key, value, kc.double(), vc.double(), slots)
    yield "slot count", (key, value, kc, vc, slots[:2])
    yield "strided slots", (key, value, kc, vc, torch.tensor([0, 9, 5, 9, -1, 9], dtype=torch.int32)[::2])
    for bad in (12, -2):
        yield f"slot {bad}", (key, value, kc, vc, torch.tensor([0, bad, -1], dtype=torch.int32))
    empty = torch.empty(0, 2, 4)
    yield "empty", (empty, empty.clone(), kc, vc, torch.empty(0, dtype=torch.int32))


def gather_cases():
    cache = torch.zeros(3, 4, 2, 4)
    table = torch.tensor([2, 0], dtype=torch.int32)
    yield "valid", (cache, table, 6)
    yield "zero length", (cache, table, 0)
    yield "negative", (cache, table, -1)
    yield "int64 table", (cache, table.to(torch.int64), 6)
    yield "2-d table", (cache, table.view(1, 2), 6)
    yield "short table", (cache, table[:1], 6)
    yield "block 3", (cache, torch.tensor([3, 0], dtype=torch.int32), 6)
    yield "block -1", (cache, torch.tensor([-1, 0], dtype=torch.int32), 6)
    yield "tail not inspected", (cache, torch.tensor([2, 0, -1], dtype=torch.int32), 6)
    yield "3-d cache", (cache[0], table, 2)
    yield "strided cache", (cache.transpose(2, 3), table, 6)
    yield "strided table", (cache, torch.tensor([2, 9, 0, 9], dtype=torch.int32)[::2], 6)


@pytest.mark.parametrize("name,args", list(store_cases()), ids=[n for n, _ in store_cases()])
def test_store_checks_match_the_validator(host, name, args):
    expected = _outcome(check_store_inputs, *args)
    assert _outcome(host.check_store, *args) == expected
    # after the checks, host tensors are refused before any launch
    if expected is None:
        with pytest.raises(ValueError, match="ROCm"):
            host.store(*args, 0)


@pytest.mark.parametrize("name,args", list(gather_cases()), ids=[n for n, _ in gather_cases()])
def test_gather_checks_match_the_validator(host, name, args):
    expected = _outcome(check_gather_inputs, *args)
    assert _outcome(host.check_gather, *args) == expected
    if expected is None:
        with pytest.raises(ValueError, match="ROCm"):
            host.gather(*args, 0)


def test_index_validation_flag_is_read_per_call(host):
    """Device-resident indexes are value-checked only under the flag (host
    tensors always); the binding reads the flag as the validator does."""
    key, value, kc, vc, _ = store_inputs()
    bad = torch.tensor([0, 12, -1], dtype=torch.int32)
    with patch.dict(os.environ, {"NANOVLLM_PAGED_KV_VALIDATE_INDICES": "0"}):
        # host tensors: checked whatever the flag says
        assert "slot outside" in _outcome(host.check_store, key, value, kc, vc, bad)


def test_build_id_matches_the_sources_and_torch(host):
    assert host.build_id() == nkv_build.host_build_id()
