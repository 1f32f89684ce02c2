"""CPU tests of the step-plan rule of the flash_attn_with_kvcache drop-in
(nanokv.flash._StepPlan): a plan serves one decode step, keyed on the
lengths tensor object, its version (where torch tracks one) and the layer
caches seen with it.  No GPU: the entries stored are placeholders."""
from __future__ import annotations

import gc

import torch

from nanokv.flash import _StepPlan


def key_of(t: torch.Tensor, block_size: int = 16):
    version = None if t.is_inference() else t._version
    return (t.data_ptr(), version, tuple(t.shape), str(t.device), block_size)


def test_one_plan_per_step_over_distinct_layer_caches():
    plans = _StepPlan()
    lengths = torch.tensor([3, 5, 7], dtype=torch.int32)
    assert plans.lookup(lengths, key_of(lengths), cache_ptr=100) is None
    plans.store(lengths, key_of(lengths), 100, "cu", 15, "plan")
    for layer_cache in (200, 300, 400):  # the step's other layers
        assert plans.lookup(lengths, key_of(lengths), layer_cache) == ("cu", 15, "plan")
    # the first layer's cache again: the next step builds a new plan
    assert plans.lookup(lengths, key_of(lengths), 100) is None


def test_in_place_update_changes_the_key():
    plans = _StepPlan()
    lengths = torch.tensor([3, 5, 7], dtype=torch.int32)
    plans.store(lengths, key_of(lengths), 100, "cu", 15, "plan")
    lengths.add_(1)  # torch bumps the version
    assert plans.lookup(lengths, key_of(lengths), 200) is None


def test_another_tensor_at_the_same_address_is_a_miss():
    """A new step's lengths may land at the freed address of the last
    step's: the entry is tied to the object itself, not to the address."""
    plans = _StepPlan()
    first = torch.tensor([3, 5, 7], dtype=torch.int32)
    plans.store(first, key_of(first), 100, "cu", 15, "plan")
    second = torch.tensor([3, 5, 7], dtype=torch.int32)
    assert plans.lookup(second, key_of(second), 200) is None
    del first
    gc.collect()
    third = torch.tensor([9, 9, 9], dtype=torch.int32)
    assert plans.lookup(third, key_of(third), 200) is None


def test_inference_tensors_rely_on_the_step_rule():
    """torch.inference_mode() tensors carry no version counter: the layer
    caches tell the steps apart."""
    plans = _StepPlan()
    with torch.inference_mode():
        lengths = torch.tensor([3, 5, 7], dtype=torch.int32)
    assert lengths.is_inference()
    plans.store(lengths, key_of(lengths), 100, "cu", 15, "plan")
    assert plans.lookup(lengths, key_of(lengths), 200) == ("cu", 15, "plan")
    assert plans.lookup(lengths, key_of(lengths), 100) is None


def test_a_different_block_size_or_shape_is_a_miss():
    plans = _StepPlan()
    lengths = torch.tensor([3, 5, 7], dtype=torch.int32)
    plans.store(lengths, key_of(lengths, 16), 100, "cu", 15, "plan")
    assert plans.lookup(lengths, key_of(lengths, 32), 200) is None
