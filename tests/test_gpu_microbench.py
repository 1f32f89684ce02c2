"""The store / gather micro-benchmark run end to end on the GPU through its
command line: a small matrix over both backends, three dtypes and the
reference's mappings, every case gated bit-exactly against the reference's
torch ops before it is timed, then the JSON and Markdown reports; and the
one-case profile replay."""
from __future__ import annotations

import json

import pytest

from nanokv import microbench as mb

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mapping", ["random_with_skips", "contiguous", "random"])
def test_matrix_run_writes_gated_reports(gpu_device, tmp_path, mapping):
    print(f"[microbench] mapping={mapping}", flush=True)
    out = tmp_path / mapping
    assert mb.main(["--backends", "hip,pytorch", "--dtypes", "float16,bfloat16,float32",
                    "--tokens", "1,257", "--kv-shapes", "1x64,8x128", "--mapping", mapping,
                    "--warmup", "3", "--iterations", "20", "--device", str(gpu_device),
                    "--output-dir", str(out)]) == 0
    report = json.loads((out / "paged-kv-microbenchmark.json").read_text())
    assert report["schema_version"] == "nanoinfer.paged_kv_benchmark.v1"
    assert report["identity"]["gpu_arch"].startswith("gfx950")
    results = report["results"]
    assert len(results) == 2 * 2 * 3 * 2 * 2
    for r in results:
        assert r["correctness"] == "pass" and len(r["samples_us"]) == 20
        assert r["latency"]["count"] == 20 and r["latency"]["p50_us"] > 0
        assert r["effective_bytes"] == mb.case_effective_bytes(mb.Case.from_selector(r["case"]["selector"]))
    text = (out / "paged-kv-microbenchmark.md").read_text()
    assert text.count("| pass |") == len(results)


def test_profile_replay_of_one_selector(gpu_device, capsys):
    selector = ("backend=hip;operation=gather;dtype=bfloat16;tokens=257;blocks=64;block=16;"
                "heads=8;dim=128;mapping=random_with_skips;seed=17")
    assert mb.main(["--case-selector", selector, "--profile-replay", "5",
                    "--device", str(gpu_device)]) == 0
    assert f"profile replay complete: {selector}" in capsys.readouterr().out
