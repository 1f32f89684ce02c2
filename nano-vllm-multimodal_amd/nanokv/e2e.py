"""End-to-end comparison of generation reports across paged-KV backends.

Restates nanovllm/benchmark/paged_kv_e2e.py:11-113 with ``hip`` among the
backends: every backend's greedy token ids must equal the ``pytorch``
backend's for every case, and latency, output throughput, peak memory and
speedup over ``pytorch`` are aggregated per backend.  The report format is
the reference's (stage ``native-sdpa`` / ``native-flash``,
``parameters.paged_kv_backend``, ``cases[*].output_token_ids`` and
``cases[*].benchmark``).
"""
from __future__ import annotations

from typing import Any, Mapping, Sequence

from nanokv.benchmark import summarize_latencies

KNOWN_BACKENDS = ("pytorch", "triton", "cuda", "hip")
BASELINE = "pytorch"


def _validate_report(backend: str, report: Mapping[str, Any]) -> list[Mapping[str, Any]]:
    if report.get("stage") not in {"native-sdpa", "native-flash"}:
        raise ValueError(f"{backend} report is not a native generation stage")
    parameters = report.get("parameters")
    if not isinstance(parameters, Mapping) or parameters.get("paged_kv_backend") != backend:
        raise ValueError(f"{backend} report has the wrong paged_kv_backend identity")
    cases = report.get("cases")
    if not isinstance(cases, list) or not cases:
        raise ValueError(f"{backend} report has no benchmark cases")
    return cases


def _tokens(cases) -> dict[str, tuple[int, ...]]:
    return {str(c["name"]): tuple(int(t) for t in c["output_token_ids"]) for c in cases}


def compare_paged_kv_reports(
    reports: Mapping[str, Mapping[str, Any]],
    backends: Sequence[str] | None = None,
) -> dict[str, Any]:
    """Compare reports keyed by backend name.  ``backends`` (default: the
    reference's trio plus ``hip`` when present) must all be reported and
    include ``pytorch``, the token reference and the speedup baseline."""
    names = tuple(backends) if backends is not None else tuple(b for b in KNOWN_BACKENDS if b in reports)
    unknown = [b for b in names if b not in KNOWN_BACKENDS]
    if unknown:
        raise ValueError(f"unknown backends: {', '.join(unknown)}")
    if BASELINE not in names or set(names) != set(reports):
        raise ValueError("reports must contain pytorch and exactly the compared backends")
    cases = {b: _validate_report(b, reports[b]) for b in names}
    reference = _tokens(cases[BASELINE])
    for backend in names:
        if backend == BASELINE:
            continue
        candidate = _tokens(cases[backend])
        if candidate != reference:
            mismatches = sorted(n for n in set(reference) | set(candidate)
                                if reference.get(n) != candidate.get(n))
            raise ValueError(f"token mismatch for backend {backend}: {', '.join(mismatches)}")
    aggregates: dict[str, dict[str, Any]] = {}
    for backend in names:
        latencies, output_tokens, peak = [], 0, 0
        for case in cases[backend]:
            bench = case.get("benchmark")
            if not isinstance(bench, Mapping):
                raise ValueError(f"{backend} case {case.get('name')} has no benchmark data")
            latencies.append(float(bench["total_latency_sec"]))
            output_tokens += int(bench["output_tokens"])
            peak = max(peak, int(bench["peak_gpu_memory_bytes"]))
        total = sum(latencies)
        summary_us = summarize_latencies(v * 1_000_000 for v in latencies)
        aggregates[backend] = {
            "case_count": len(latencies),
            "total_latency_sec": total,
            "output_tokens": output_tokens,
            "output_tokens_per_sec": output_tokens / total if total else 0.0,
            "peak_gpu_memory_bytes": peak,
            "case_latency_sec": {
                k.replace("_us", "_sec"): (v / 1_000_000 if k.endswith("_us") else v)
                for k, v in summary_us.items()
            },
        }
    baseline = aggregates[BASELINE]["total_latency_sec"]
    for backend in names:
        latency = aggregates[backend]["total_latency_sec"]
        aggregates[backend]["speedup_vs_pytorch"] = baseline / latency if latency else None
    return {
        "schema_version": "nanoinfer.paged_kv_e2e_comparison.v1",
        "tokens_exact": True,
        "case_names": list(reference),
        "backends": aggregates,
    }


def render_paged_kv_e2e_markdown(result: Mapping[str, Any]) -> str:
    lines = [
        "# Paged KV End-to-End Comparison",
        "",
        f"Greedy token IDs exact across all backends: `{str(result['tokens_exact']).lower()}`",
        "",
        "| Backend | Cases | Total latency (s) | Output tok/s | P50 case (s) | P95 case (s) | "
        "P99 case (s) | Peak GiB | Speedup |",
        "|---|---:|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for backend, values in result["backends"].items():
        latency = values["case_latency_sec"]
        speedup = values["speedup_vs_pytorch"]
        lines.append(
            f"| {backend} | {values['case_count']} | {values['total_latency_sec']:.6f} | "
            f"{values['output_tokens_per_sec']:.3f} | {latency['p50_sec']:.6f} | "
            f"{latency['p95_sec']:.6f} | {latency['p99_sec']:.6f} | "
            f"{values['peak_gpu_memory_bytes'] / 1024**3:.3f} | "
            + ("n/a |" if speedup is None else f"{speedup:.3f}x |")
        )
    return "\n".join(lines) + "\n"
