"""CPU tests of the store / gather micro-benchmark (nanokv.microbench): the
command line, the case matrix and selectors, the reference's byte count, the
correctness gate's order and the atomic report files.  The known answers
are the reference's own (tests/test_bench_paged_kv.py:21-140), with the hip
and pytorch backends this platform builds."""
from __future__ import annotations

import json
import os

import pytest
import torch

from nanokv import microbench as mb


def test_cli_defaults_are_the_reference_matrix_and_take_a_replay():
    args = mb.build_parser().parse_args([])
    assert args.operations == ("store", "gather") and args.dtypes == ("float16", "bfloat16")
    assert args.tokens == (1, 8, 257) and args.kv_shapes == ((1, 64), (2, 128), (8, 128))
    assert (args.num_blocks, args.block_size, args.mapping, args.seed) == (64, 16, "random_with_skips", 17)
    assert (args.warmup, args.iterations) == (100, 1000)
    selector = ("backend=hip;operation=store;dtype=float16;tokens=257;blocks=64;block=16;"
                "heads=8;dim=128;mapping=random;seed=17")
    args = mb.build_parser().parse_args(["--case-selector", selector, "--profile-replay", "25"])
    assert (args.case_selector, args.profile_replay) == (selector, 25)
    assert mb.resolve_cases(args) == (mb.Case("hip", "store", torch.float16, 257, 64, 16, 8, 128,
                                              "random", 17),)


@pytest.mark.parametrize("flag,value", [("--tokens", "1,0"), ("--tokens", "a"), ("--kv-shapes", "8"),
                                        ("--kv-shapes", "0x64"), ("--kv-shapes", "2y128"),
                                        ("--backends", ",")])
def test_cli_rejects_bad_lists(flag, value):
    with pytest.raises(SystemExit):
        mb.build_parser().parse_args([flag, value])


def test_matrix_is_deterministic_unique_and_in_the_reference_order():
    kwargs = dict(backends=("hip", "pytorch"), operations=("store", "gather"),
                  dtypes=(torch.float16,), token_counts=(1, 257), kv_shapes=((2, 128),),
                  block_size=16, num_blocks=32)
    first, second = mb.expand_matrix(**kwargs), mb.expand_matrix(**kwargs)
    assert first == second and len(first) == 8 and len({c.selector for c in first}) == 8
    assert [(c.backend, c.operation, c.num_tokens) for c in first[:3]] == [
        ("hip", "store", 1), ("hip", "store", 257), ("hip", "gather", 1)]


def test_selector_round_trips_and_rejects_malformed_ones():
    case = mb.Case("hip", "gather", torch.bfloat16, 257, 64, 16, 8, 80, "random_with_skips", 19)
    assert mb.Case.from_selector(case.selector) == case
    assert case.to_dict()["selector"] == case.selector and case.to_dict()["dtype"] == "bfloat16"
    bad = [case.selector.replace(";seed=19", ""), case.selector + ";extra=1",
           case.selector.replace("bfloat16", "int8"), case.selector.replace("tokens=257", "tokens=x"),
           case.selector.replace("seed=19", "seed=19;seed=20")]
    for selector in bad:
        with pytest.raises(ValueError, match="invalid Paged KV case selector"):
            mb.Case.from_selector(selector)


def test_cases_are_validated():
    with pytest.raises(ValueError, match="not built on this platform"):
        mb.Case("cuda", "store", torch.float16, 8, 4, 16, 2, 128)
    with pytest.raises(ValueError, match="capacity"):
        mb.Case("hip", "store", torch.float16, 65, 4, 16, 2, 128)
    with pytest.raises(ValueError, match="positive"):
        mb.Case("hip", "gather", torch.float16, 8, 4, 16, 0, 128)
    with pytest.raises(ValueError, match="slot mapping"):
        mb.Case("hip", "store", torch.float16, 8, 4, 16, 2, 128, "sorted")


def test_effective_bytes_counts_payload_reads_and_writes():
    store = mb.Case("hip", "store", torch.float16, 8, 4, 16, 2, 128)
    gather = mb.Case("pytorch", "gather", torch.float32, 9, 4, 16, 1, 80)
    assert mb.case_effective_bytes(store) == 8 * 2 * 128 * 2 * 4
    assert mb.case_effective_bytes(gather) == 9 * 1 * 80 * 4 * 2


def test_correctness_gate_runs_before_warmup_and_timing():
    calls = []
    got = mb.gated(lambda: calls.append("check"), lambda: calls.append("warmup"),
                   lambda: calls.append("measure") or [1.0, 2.0])
    assert calls == ["check", "warmup", "measure"] and got == [1.0, 2.0]
    calls.clear()

    def failing():
        calls.append("check")
        raise AssertionError("differs")

    with pytest.raises(AssertionError):
        mb.gated(failing, lambda: calls.append("warmup"), lambda: calls.append("measure") or [])
    assert calls == ["check"]


def test_atomic_reports_round_trip_and_never_leave_partial_files(tmp_path, monkeypatch):
    case = mb.Case("pytorch", "store", torch.float16, 1, 2, 16, 1, 64)
    report = {"schema_version": mb.SCHEMA, "identity": {"gpu_uuid": "GPU-test"},
              "results": [{"case": case.to_dict(), "correctness": "pass", "latency": {
                  "p50_us": 1.5, "p95_us": 2.0, "p99_us": 2.1}, "effective_gbps_at_p50": 0.1,
                  "samples_us": [1.25, 1.5]}]}
    path = tmp_path / "out" / "report.json"
    mb.write_json_atomic(path, report)
    assert json.loads(path.read_text()) == report
    assert report["schema_version"] == "nanoinfer.paged_kv_benchmark.v1"

    def broken_replace(src, dst):
        raise OSError("disk gone")

    monkeypatch.setattr(os, "replace", broken_replace)
    with pytest.raises(OSError):
        mb.write_json_atomic(path, {"schema_version": "other"})
    assert json.loads(path.read_text()) == report          # the old file is whole
    assert sorted(p.name for p in path.parent.iterdir()) == ["report.json"]  # no temporary left
    text = mb.render_markdown(report)
    assert "| pytorch | store | float16 | 1 | 1x64 | contiguous | 1.50 |" in text


def test_profile_replay_needs_one_selector():
    with pytest.raises(ValueError, match="--case-selector"):
        mb.main(["--profile-replay", "3"])
