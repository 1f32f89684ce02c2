"""CPU tests of the benchmark plumbing: byte accounting, percentiles, the
CPU-baseline leg and the one-GPU guard of bench.py."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from nanokv import benchmark, workloads

REPO = Path(__file__).resolve().parents[1]


def test_latency_summary_matches_reference_definition():
    summary = benchmark.summarize_latencies([1.0, 2.0, 3.0, 4.0])
    assert summary["count"] == 4
    assert summary["p50_us"] == 2.5
    assert summary["p95_us"] == pytest.approx(3.85)
    assert summary["p99_us"] == pytest.approx(3.97)
    with pytest.raises(ValueError):
        benchmark.summarize_latencies([])


def test_effective_bytes_matches_reference_known_answers():
    assert benchmark.effective_bytes("store", 8, 2, 128, 2) == 8 * 2 * 128 * 2 * 4
    assert benchmark.effective_bytes("gather", 9, 1, 80, 4) == 9 * 80 * 4 * 2


def test_algorithmic_bytes_closed_forms():
    wl = workloads.build("decode_store")
    valid = int((wl.slot_mapping >= 0).sum())
    assert valid == 60
    assert wl.store_bytes() == 60 * 4 * 2048 + 4 * 64 == 491_776
    wl = workloads.build("chunked_prefill")
    assert wl.store_bytes() == 8192 * 4 * 2048 + 4 * 8192
    lens = wl.context_lens.astype(np.int64)
    blocks = int(((lens + 255) // 256).sum())
    assert wl.gather_bytes() == int(lens.sum()) * 4 * 2048 + 8 * blocks + 4 * 17


def test_cpu_baselines_run_on_a_small_step():
    sys.path.insert(0, str(REPO))
    import bench

    wl = workloads.build("decode_step", num_layers=2, num_live=8, churn=2, max_ctx=1024)
    result = bench.cpu_reference_baseline(wl, 2, [], runs=3)
    assert result["kind"] == "port" and result["unit"] == "GB/s"
    runs = result["seconds_per_layer_runs"]
    assert len(runs) == 3 and result["seconds_per_layer"] == sorted(runs)[1]
    assert "median of 3 runs" in result["sample"]
    assert result["value"] > 0 and result["cores"] >= 1 and result["torch_threads"] == result["cores"]
    assert "index_copy_" in result["ops"] and result["cpu_model"]
    port = bench.openmp_port_baseline(wl, layers=2, repeats=1)
    assert port["kind"] == "port" and port["value"] > 0


def test_reference_torch_ops_on_host_equal_the_oracle():
    """The CPU baseline times TorchReferenceBackend on host tensors; on the
    same inputs it must compute what the oracle computes."""
    import torch

    from oracle import paged_kv as oracle

    ref = benchmark.TorchReferenceBackend()
    g = torch.Generator().manual_seed(3)
    kc = torch.randn((6, 4, 2, 8), generator=g).to(torch.bfloat16)
    vc = torch.randn((6, 4, 2, 8), generator=g).to(torch.bfloat16)
    key = torch.randn((5, 2, 8), generator=g).to(torch.bfloat16)
    value = torch.randn((5, 2, 8), generator=g).to(torch.bfloat16)
    slots = torch.tensor([3, -1, 17, 0, 22], dtype=torch.int32)
    hk, hv = kc.view(torch.int16).numpy().copy(), vc.view(torch.int16).numpy().copy()
    oracle.store(key.view(torch.int16).numpy(), value.view(torch.int16).numpy(), hk, hv, slots.numpy())
    ref.store(key, value, kc, vc, slots)
    assert np.array_equal(kc.view(torch.int16).numpy(), hk)
    assert np.array_equal(vc.view(torch.int16).numpy(), hv)
    table = torch.tensor([5, 0, 2], dtype=torch.int32)
    got = ref.gather(kc, table, 10).view(torch.int16).numpy()
    assert np.array_equal(got, oracle.gather(hk, table.numpy(), 10))


def test_environment_identity_fields():
    identity = benchmark.environment_identity()
    for key in ("timestamp_utc", "torch", "hip_status", "cpu_model", "host_threads", "platform"):
        assert key in identity
    assert identity["host_threads"] >= 1


def test_bench_rejects_a_case_without_replay():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--case", "chunked_prefill"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2 and "--profile-replay" in proc.stderr


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "8"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
