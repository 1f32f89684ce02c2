"""CPU tests of the plugin API: validation contract, index-validation flag,
backend-name resolution and construction, mirroring the reference's
tests/test_paged_kv_backends.py:26-124 and tests/test_paged_kv_cuda.py:
162-169 (names without eager compilation)."""
from __future__ import annotations

import os
import unittest
from types import SimpleNamespace
from unittest.mock import patch

import torch

from nanokv.paged_kv import (
    create_paged_kv_backend,
    index_value_validation_enabled,
    resolve_paged_kv_backend_name,
    validate_gather_inputs,
    validate_store_inputs,
)


def store_inputs():
    key = torch.arange(3 * 2 * 4, dtype=torch.float32).reshape(3, 2, 4)
    value = key + 100
    key_cache = torch.full((3, 4, 2, 4), -1.0)
    value_cache = torch.full_like(key_cache, -1.0)
    slots = torch.tensor([0, 5, -1], dtype=torch.int32)
    return key, value, key_cache, value_cache, slots


class ValidationTests(unittest.TestCase):
    def test_gpu_index_value_validation_is_debug_opt_in(self):
        cuda_tensor = SimpleNamespace(is_cuda=True)
        cpu_tensor = SimpleNamespace(is_cuda=False)
        with patch.dict(os.environ, {}, clear=False):
            os.environ.pop("NANOVLLM_PAGED_KV_VALIDATE_INDICES", None)
            self.assertFalse(index_value_validation_enabled(cuda_tensor))
            self.assertTrue(index_value_validation_enabled(cpu_tensor))
        for flag in ("1", "true", "YES", " on "):
            with patch.dict(os.environ, {"NANOVLLM_PAGED_KV_VALIDATE_INDICES": flag}):
                self.assertTrue(index_value_validation_enabled(cuda_tensor))
        with patch.dict(os.environ, {"NANOVLLM_PAGED_KV_VALIDATE_INDICES": "0"}):
            self.assertFalse(index_value_validation_enabled(cuda_tensor))

    def test_valid_store_contract_returns_dimensions(self):
        dims = validate_store_inputs(*store_inputs())
        self.assertEqual((dims.num_tokens, dims.num_kv_heads, dims.head_dim), (3, 2, 4))
        self.assertEqual(dims.num_slots, 12)

    def test_store_rejects_shape_dtype_and_layout_mismatches(self):
        key, value, key_cache, value_cache, slots = store_inputs()
        cases = [
            ((key[:2], value, key_cache, value_cache, slots), "matching shape"),
            ((key, value, key_cache[:, :, :1], value_cache, slots), "cache shape"),
            ((key, value, key_cache, value_cache, slots.to(torch.int64)), "int32"),
            ((key.transpose(1, 2), value.transpose(1, 2), key_cache, value_cache, slots), "inner dimensions"),
            ((key, value.to(torch.float16), key_cache, value_cache, slots), "matching shape|dtype"),
            ((key, value, key_cache, value_cache, slots[:2]), "length"),
        ]
        for arguments, message in cases:
            with self.subTest(message=message):
                with self.assertRaisesRegex(ValueError, message):
                    validate_store_inputs(*arguments)

    def test_store_rejects_non_contiguous_slots(self):
        key, value, key_cache, value_cache, _ = store_inputs()
        slots = torch.tensor([0, 9, 5, 9, -1, 9], dtype=torch.int32)[::2]
        with self.assertRaisesRegex(ValueError, "contiguous"):
            validate_store_inputs(key, value, key_cache, value_cache, slots)

    def test_store_rejects_out_of_range_slots_but_accepts_minus_one(self):
        key, value, key_cache, value_cache, slots = store_inputs()
        validate_store_inputs(key, value, key_cache, value_cache, slots)
        for bad in (12, -2):
            slots = torch.tensor([0, bad, -1], dtype=torch.int32)
            with self.assertRaisesRegex(ValueError, "slot"):
                validate_store_inputs(key, value, key_cache, value_cache, slots)

    def test_gather_validates_length_table_and_dtype(self):
        cache = torch.zeros(3, 4, 2, 4)
        table = torch.tensor([2, 0], dtype=torch.int32)
        self.assertEqual(validate_gather_inputs(cache, table, 6).required_blocks, 2)
        self.assertEqual(validate_gather_inputs(cache, table, 0).required_blocks, 0)
        with self.assertRaisesRegex(ValueError, "non-negative"):
            validate_gather_inputs(cache, table, -1)
        with self.assertRaisesRegex(ValueError, "int32"):
            validate_gather_inputs(cache, table.to(torch.int64), 6)
        with self.assertRaisesRegex(ValueError, "cover"):
            validate_gather_inputs(cache, table[:1], 6)
        with self.assertRaisesRegex(ValueError, "physical block"):
            validate_gather_inputs(cache, torch.tensor([3, 0], dtype=torch.int32), 6)
        with self.assertRaisesRegex(ValueError, "physical block"):
            validate_gather_inputs(cache, torch.tensor([-1, 0], dtype=torch.int32), 6)
        # entries past the required blocks are not inspected
        validate_gather_inputs(cache, torch.tensor([2, 0, -1], dtype=torch.int32), 6)
        with self.assertRaisesRegex(ValueError, "shape"):
            validate_gather_inputs(cache[0], table, 2)


class BackendResolutionTests(unittest.TestCase):
    def test_explicit_backends_are_preserved(self):
        for name in ("pytorch", "triton", "cuda", "hip"):
            self.assertEqual(
                resolve_paged_kv_backend_name(name, cuda_available=True, cuda_extension_available=True),
                name,
            )

    def test_auto_prefers_hip_then_reference_order(self):
        self.assertEqual(
            resolve_paged_kv_backend_name(
                "auto", cuda_available=True, cuda_extension_available=False,
                hip_available=True, hip_extension_available=True),
            "hip",
        )
        self.assertEqual(
            resolve_paged_kv_backend_name(
                "auto", cuda_available=True, cuda_extension_available=True,
                hip_available=True, hip_extension_available=False),
            "cuda",
        )
        self.assertEqual(
            resolve_paged_kv_backend_name("auto", cuda_available=True, cuda_extension_available=False),
            "triton",
        )
        self.assertEqual(
            resolve_paged_kv_backend_name("auto", cuda_available=False, cuda_extension_available=False),
            "pytorch",
        )

    def test_invalid_backend_is_rejected(self):
        with self.assertRaisesRegex(ValueError, "paged_kv_backend"):
            resolve_paged_kv_backend_name("flash", cuda_available=True, cuda_extension_available=True)

    def test_hip_backend_has_stable_name_without_loading(self):
        backend = create_paged_kv_backend("hip")
        self.assertEqual(backend.name, "hip")

    def test_host_engine_backends_and_unknown_names_raise(self):
        for name in ("pytorch", "triton", "cuda"):
            with self.assertRaisesRegex(ValueError, "host engine"):
                create_paged_kv_backend(name)
        with self.assertRaisesRegex(ValueError, "unknown paged KV backend"):
            create_paged_kv_backend("flash")

    def test_hip_backend_rejects_cpu_tensors_after_validation(self):
        backend = create_paged_kv_backend("hip")
        with self.assertRaisesRegex(ValueError, "ROCm"):
            backend.store(*store_inputs())
        with self.assertRaisesRegex(ValueError, "ROCm"):
            backend.gather(torch.zeros(3, 4, 2, 4), torch.tensor([2, 0], dtype=torch.int32), 6)
        with self.assertRaisesRegex(ValueError, "ROCm|cuda"):
            backend.allocate((2, 1, 4, 2, 4), dtype=torch.bfloat16, device="cpu")
        with self.assertRaisesRegex(ValueError, "dtype"):
            backend.allocate((2, 1, 4, 2, 4), dtype=torch.int8, device="cuda")

    def test_legacy_store_kvcache_keeps_signature_and_contract(self):
        import inspect

        from nanokv.paged_kv import store_kvcache

        # attention.py:10-16: store_kvcache(key, value, k_cache, v_cache, slot_mapping)
        self.assertEqual(len(inspect.signature(store_kvcache).parameters), 5)
        key, value, key_cache, value_cache, slots = store_inputs()
        with self.assertRaisesRegex(ValueError, "matching shape"):
            store_kvcache(key[:2], value, key_cache, value_cache, slots)
        with self.assertRaisesRegex(ValueError, "ROCm"):
            store_kvcache(key, value, key_cache, value_cache, slots)


if __name__ == "__main__":
    unittest.main()
