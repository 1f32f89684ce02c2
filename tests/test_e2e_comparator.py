"""CPU tests of the end-to-end comparator (nanokv.e2e): token exactness
against the pytorch backend with the first diverging token per case,
per-backend aggregates, report validation and the command line.  Expected
aggregates are worked out by hand in each test."""
from __future__ import annotations

import json

import pytest

from nanokv.e2e import (
    compare_paged_kv_reports,
    first_divergence,
    main,
    parse_run,
    render_paged_kv_e2e_markdown,
)

PROMPTS = {  # case name -> greedy tokens of the oracle backend
    "describe-image": (151644, 872, 198, 785, 2168),
    "two-images": (40, 1079, 11),
    "text-only": (9707,),
}


def generation_report(backend, seconds, *, stage="native-flash", tokens=None, peak_gib=1.0):
    """A report as the engine's generation benchmark writes it: the case
    latencies in ``seconds`` (one per prompt, in PROMPTS order)."""
    tokens = tokens or PROMPTS
    return {
        "stage": stage,
        "parameters": {"paged_kv_backend": backend, "max_tokens": 64},
        "cases": [
            {"name": name, "output_token_ids": list(ids),
             "benchmark": {"total_latency_sec": s, "output_tokens": len(ids),
                           "peak_gpu_memory_bytes": int(peak_gib * 2**30) + k}}
            for k, ((name, ids), s) in enumerate(zip(tokens.items(), seconds))
        ],
    }


def test_aggregates_and_speedups_over_the_oracle_backend():
    result = compare_paged_kv_reports({
        "pytorch": generation_report("pytorch", (3.0, 2.0, 1.0)),
        "hip": generation_report("hip", (0.5, 0.25, 0.25), peak_gib=2.0),
        "cuda": generation_report("cuda", (1.0, 1.0, 1.0)),
    })
    assert result["tokens_exact"] and result["divergences"] == {}
    assert result["case_names"] == list(PROMPTS)
    hip = result["backends"]["hip"]
    assert hip["total_latency_sec"] == pytest.approx(1.0)
    assert hip["output_tokens"] == 9
    assert hip["output_tokens_per_sec"] == pytest.approx(9.0)
    assert hip["speedup_vs_pytorch"] == pytest.approx(6.0)
    assert hip["peak_gpu_memory_bytes"] == 2 * 2**30 + 2
    assert hip["case_latency_sec"]["p50_sec"] == pytest.approx(0.25)
    assert hip["case_latency_sec"]["max_sec"] == pytest.approx(0.5)
    assert result["backends"]["cuda"]["speedup_vs_pytorch"] == pytest.approx(2.0)
    assert result["backends"]["pytorch"]["speedup_vs_pytorch"] == pytest.approx(1.0)
    text = render_paged_kv_e2e_markdown(result)
    assert "| hip | native-flash | 3 |" in text and "6.00x" in text


def test_first_divergence_positions():
    assert first_divergence((1, 2, 3), (1, 2, 3)) is None
    assert first_divergence((1, 2, 3), (1, 7, 3))["index"] == 1
    shorter = first_divergence((1, 2, 3), (1, 2))
    assert (shorter["index"], shorter["expected"], shorter["got"]) == (2, 3, None)
    longer = first_divergence((), (5,))
    assert (longer["index"], longer["expected"], longer["got"]) == (0, None, 5)


def test_token_fork_names_case_and_position():
    forked = dict(PROMPTS, **{"two-images": (40, 1079, 13)})
    reports = {"pytorch": generation_report("pytorch", (1, 1, 1)),
               "hip": generation_report("hip", (1, 1, 1), tokens=forked)}
    with pytest.raises(ValueError, match=r"token mismatch for backend hip: two-images "
                                         r"\(first differs at token 2: 11 != 13\)"):
        compare_paged_kv_reports(reports)
    result = compare_paged_kv_reports(reports, require_exact=False)
    assert not result["tokens_exact"]
    assert result["divergences"] == {"hip": {"two-images": {
        "index": 2, "expected": 11, "got": 13, "expected_length": 3, "got_length": 3}}}
    assert "| two-images | 2 | 11 | 13 |" in render_paged_kv_e2e_markdown(result)


def test_missing_case_counts_as_divergence():
    partial = {k: v for k, v in PROMPTS.items() if k != "text-only"}
    with pytest.raises(ValueError, match=r"text-only \(missing in hip\)"):
        compare_paged_kv_reports({"pytorch": generation_report("pytorch", (1, 1, 1)),
                                  "hip": generation_report("hip", (1, 1), tokens=partial)})


def test_report_problems_are_listed_together():
    bad = generation_report("cuda", (1, 1, 1), stage="hf")
    del bad["cases"][1]["benchmark"]["output_tokens"]
    with pytest.raises(ValueError) as info:
        compare_paged_kv_reports({"pytorch": generation_report("pytorch", (1, 1, 1)), "hip": bad})
    message = str(info.value)
    assert "stage 'hf'" in message and "identifies paged_kv_backend 'cuda'" in message
    assert "lacks output_tokens" in message
    with pytest.raises(ValueError, match="needs a pytorch report"):
        compare_paged_kv_reports({"hip": generation_report("hip", (1, 1, 1))})
    with pytest.raises(ValueError, match="unknown backends: flash"):
        compare_paged_kv_reports({"pytorch": generation_report("pytorch", (1, 1, 1))},
                                 backends=("pytorch", "flash"))
    empty = generation_report("hip", ())
    with pytest.raises(ValueError, match="no benchmark cases"):
        parse_run("hip", empty)


def test_command_line_writes_json_and_markdown(tmp_path, capsys):
    paths = {}
    for name, seconds in (("pytorch", (2, 2, 2)), ("hip", (1, 0.5, 0.5))):
        paths[name] = tmp_path / f"{name}.json"
        paths[name].write_text(json.dumps(generation_report(name, seconds)))
    out = tmp_path / "cmp"
    assert main(["--pytorch", str(paths["pytorch"]), "--report", f"hip={paths['hip']}",
                 "--output-dir", str(out)]) == 0
    saved = json.loads((out / "paged-kv-e2e-comparison.json").read_text())
    assert saved["backends"]["hip"]["speedup_vs_pytorch"] == pytest.approx(3.0)
    assert (out / "paged-kv-e2e-comparison.md").read_text() in capsys.readouterr().out

    forked = dict(PROMPTS, **{"text-only": (9708,)})
    paths["hip"].write_text(json.dumps(generation_report("hip", (1, 1, 1), tokens=forked)))
    assert main(["--pytorch", str(paths["pytorch"]), "--hip", str(paths["hip"]),
                 "--output-dir", str(out), "--allow-divergence"]) == 1
    assert json.loads((out / "paged-kv-e2e-comparison.json").read_text())["divergences"]
    with pytest.raises(SystemExit):
        main(["--hip", str(paths["hip"])])


def test_negative_or_missing_latency_is_rejected_and_schema_is_the_reference_id():
    """A negative (or non-numeric) case latency is a report problem, as the
    reference's latency summary rejects negative samples
    (benchmark/paged_kv.py:202-205); the result carries the reference's
    schema id (paged_kv_e2e.py:87), whose field names it uses."""
    for latency in (-0.5, "fast", None):
        bad = generation_report("hip", (1.0, latency, 2.0))
        with pytest.raises(ValueError, match="'two-images' total_latency_sec must be a non-negative"):
            parse_run("hip", bad)
    result = compare_paged_kv_reports({"pytorch": generation_report("pytorch", (1.0, 2.0, 0.0)),
                                       "hip": generation_report("hip", (0.5, 1.0, 0.0))})
    assert result["schema_version"] == "nanoinfer.paged_kv_e2e_comparison.v1"
