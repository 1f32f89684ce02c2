"""CPU tests of the end-to-end comparator, mirroring the reference's
tests/test_paged_kv_e2e.py:7-59 with the hip backend added."""
from __future__ import annotations

import pytest

from nanokv.e2e import compare_paged_kv_reports, render_paged_kv_e2e_markdown


def report(backend, latencies=(1.0, 2.0), tokens=((1, 2), (3, 4, 5))):
    return {
        "stage": "native-sdpa",
        "parameters": {"paged_kv_backend": backend},
        "cases": [
            {
                "name": f"case-{index}",
                "output_token_ids": list(token_ids),
                "benchmark": {
                    "total_latency_sec": latency,
                    "output_tokens": len(token_ids),
                    "peak_gpu_memory_bytes": 100 + index,
                },
            }
            for index, (latency, token_ids) in enumerate(zip(latencies, tokens))
        ],
    }


def test_compares_exact_tokens_latency_throughput_and_memory():
    result = compare_paged_kv_reports({
        "pytorch": report("pytorch", latencies=(2.0, 4.0)),
        "triton": report("triton", latencies=(1.0, 2.0)),
        "cuda": report("cuda", latencies=(0.5, 1.0)),
    })
    assert result["tokens_exact"]
    assert result["backends"]["pytorch"]["total_latency_sec"] == 6.0
    assert result["backends"]["cuda"]["output_tokens_per_sec"] == pytest.approx(5 / 1.5)
    assert result["backends"]["cuda"]["speedup_vs_pytorch"] == 4.0
    assert result["backends"]["cuda"]["peak_gpu_memory_bytes"] == 101


def test_hip_joins_the_comparison():
    result = compare_paged_kv_reports({
        "pytorch": report("pytorch", latencies=(2.0, 4.0)),
        "hip": report("hip", latencies=(0.25, 0.5)),
    })
    assert result["backends"]["hip"]["speedup_vs_pytorch"] == 8.0
    assert "| hip | 2 |" in render_paged_kv_e2e_markdown(result)


def test_rejects_any_backend_token_difference():
    with pytest.raises(ValueError, match="token mismatch for backend hip"):
        compare_paged_kv_reports({
            "pytorch": report("pytorch"),
            "hip": report("hip", tokens=((1, 9), (3, 4, 5))),
        })


def test_rejects_wrong_identity_missing_baseline_and_empty_cases():
    with pytest.raises(ValueError, match="identity"):
        compare_paged_kv_reports({"pytorch": report("pytorch"), "hip": report("cuda")})
    with pytest.raises(ValueError, match="pytorch"):
        compare_paged_kv_reports({"hip": report("hip")})
    empty = report("hip")
    empty["cases"] = []
    with pytest.raises(ValueError, match="no benchmark cases"):
        compare_paged_kv_reports({"pytorch": report("pytorch"), "hip": empty})
    with pytest.raises(ValueError, match="unknown backends"):
        compare_paged_kv_reports({"pytorch": report("pytorch")}, backends=("pytorch", "flash"))
