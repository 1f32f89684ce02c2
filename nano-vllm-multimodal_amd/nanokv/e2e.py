"""Token-exactness and speed comparison of generation runs across paged-KV
backends, with a command line.

What it answers (the role of the reference's
nanovllm/benchmark/paged_kv_e2e.py:23-91 and compare_paged_kv_e2e.py:15-52):
given one generation report per backend for the same prompts, does every
backend emit the same greedy tokens as the ``pytorch`` backend (the
oracle backend), and how do latency, output throughput and peak memory
compare?  The input and output field names are the reference's, so its
generation reports can be fed in unchanged and its consumers can read the
result; the structure of the comparison is this module's own:

* each report is parsed once into a :class:`Run` (typed cases keyed by
  name), with the problems of every report collected before anything is
  raised;
* tokens are compared case by case and the first diverging position is
  recorded (index, the oracle's token, the backend's token, or the shorter
  length), so a mismatch says where decoding forked, not only which case;
* per-backend aggregates come from one pass over the parsed cases.

Input report (one per backend)::

    {"stage": "native-sdpa" | "native-flash",
     "parameters": {"paged_kv_backend": <backend>},
     "cases": [{"name": str, "output_token_ids": [int, ...],
                "benchmark": {"total_latency_sec": float,
                              "output_tokens": int,
                              "peak_gpu_memory_bytes": int}}, ...]}

Command line::

    python -m nanokv.e2e --pytorch p.json --hip h.json [--cuda c.json]
        [--triton t.json] [--report NAME=PATH ...] [--output-dir DIR]
        [--allow-divergence]
"""
from __future__ import annotations

import argparse
import json
import os
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterable, Mapping

from nanokv.benchmark import linear_percentile

ORACLE_BACKEND = "pytorch"
BACKEND_NAMES = ("pytorch", "triton", "cuda", "hip")
GENERATION_STAGES = ("native-sdpa", "native-flash")
# The reference's schema id (paged_kv_e2e.py:87): the result carries the
# reference's field names, so a consumer that keys on the id reads it.
SCHEMA = "nanoinfer.paged_kv_e2e_comparison.v1"


@dataclass(frozen=True)
class Case:
    tokens: tuple[int, ...]
    latency_sec: float
    output_tokens: int
    peak_bytes: int


@dataclass(frozen=True)
class Run:
    backend: str
    stage: str
    cases: dict[str, Case]  # insertion order = report order


def _problems_of(backend: str, report: Any) -> list[str]:
    """Everything wrong with one report, as messages (empty if usable)."""
    if not isinstance(report, Mapping):
        return [f"{backend}: report is not a JSON object"]
    found = []
    if report.get("stage") not in GENERATION_STAGES:
        found.append(f"{backend}: stage {report.get('stage')!r} is not a native generation "
                     f"stage ({', '.join(GENERATION_STAGES)})")
    claimed = (report.get("parameters") or {}).get("paged_kv_backend") \
        if isinstance(report.get("parameters"), Mapping) else None
    if claimed != backend:
        found.append(f"{backend}: report identifies paged_kv_backend {claimed!r}")
    cases = report.get("cases")
    if not isinstance(cases, list) or not cases:
        found.append(f"{backend}: no benchmark cases")
        return found
    names = [c.get("name") if isinstance(c, Mapping) else None for c in cases]
    if len(set(map(str, names))) != len(names):
        found.append(f"{backend}: case names repeat")
    for name, case in zip(names, cases):
        if not isinstance(case, Mapping) or not isinstance(case.get("output_token_ids"), list):
            found.append(f"{backend}: case {name!r} has no output_token_ids")
        elif not isinstance(case.get("benchmark"), Mapping):
            found.append(f"{backend}: case {name!r} has no benchmark data")
        else:
            missing = [k for k in ("total_latency_sec", "output_tokens", "peak_gpu_memory_bytes")
                       if k not in case["benchmark"]]
            if missing:
                found.append(f"{backend}: case {name!r} benchmark lacks {', '.join(missing)}")
                continue
            try:
                latency = float(case["benchmark"]["total_latency_sec"])
            except (TypeError, ValueError):
                latency = float("nan")
            # the reference's latency summary rejects negative samples
            # (benchmark/paged_kv.py:202-205)
            if not latency >= 0.0:
                found.append(f"{backend}: case {name!r} total_latency_sec must be a "
                             f"non-negative number, got {case['benchmark']['total_latency_sec']!r}")
    return found


def parse_run(backend: str, report: Mapping[str, Any]) -> Run:
    """One backend's report as a :class:`Run`; ValueError lists every
    problem of the report."""
    problems = _problems_of(backend, report)
    if problems:
        raise ValueError("invalid report: " + "; ".join(problems))
    cases = {}
    for raw in report["cases"]:
        bench = raw["benchmark"]
        cases[str(raw["name"])] = Case(
            tokens=tuple(int(t) for t in raw["output_token_ids"]),
            latency_sec=float(bench["total_latency_sec"]),
            output_tokens=int(bench["output_tokens"]),
            peak_bytes=int(bench["peak_gpu_memory_bytes"]),
        )
    return Run(backend, str(report["stage"]), cases)


def first_divergence(expected: tuple[int, ...], got: tuple[int, ...]) -> dict[str, Any] | None:
    """Where ``got`` leaves ``expected``: the first index whose tokens
    differ, or where the shorter sequence ends; None if they are equal."""
    if expected == got:
        return None
    shared = min(len(expected), len(got))
    index = next((i for i in range(shared) if expected[i] != got[i]), shared)
    return {
        "index": index,
        "expected": expected[index] if index < len(expected) else None,
        "got": got[index] if index < len(got) else None,
        "expected_length": len(expected),
        "got_length": len(got),
    }


def _divergences(oracle: Run, other: Run) -> dict[str, dict[str, Any]]:
    found = {}
    for name in list(oracle.cases) + [n for n in other.cases if n not in oracle.cases]:
        if name not in other.cases:
            found[name] = {"missing_in": other.backend}
        elif name not in oracle.cases:
            found[name] = {"missing_in": oracle.backend}
        else:
            fork = first_divergence(oracle.cases[name].tokens, other.cases[name].tokens)
            if fork is not None:
                found[name] = fork
    return found


def _aggregate(run: Run) -> dict[str, Any]:
    latencies = [c.latency_sec for c in run.cases.values()]
    total = sum(latencies)
    tokens = sum(c.output_tokens for c in run.cases.values())
    spread = {f"p{q}_sec": linear_percentile(latencies, q / 100) for q in (50, 95, 99)}
    spread.update(count=len(latencies), mean_sec=total / len(latencies), min_sec=min(latencies),
                  max_sec=max(latencies))
    return {
        "stage": run.stage,
        "case_count": len(latencies),
        "total_latency_sec": total,
        "output_tokens": tokens,
        "output_tokens_per_sec": tokens / total if total > 0 else 0.0,
        "peak_gpu_memory_bytes": max(c.peak_bytes for c in run.cases.values()),
        "case_latency_sec": spread,
    }


def _describe(backend: str, divergences: Mapping[str, Mapping[str, Any]]) -> str:
    parts = []
    for name, d in divergences.items():
        if "missing_in" in d:
            parts.append(f"{name} (missing in {d['missing_in']})")
        else:
            parts.append(f"{name} (first differs at token {d['index']}: "
                         f"{d['expected']} != {d['got']})")
    return f"token mismatch for backend {backend}: " + ", ".join(parts)


def compare_paged_kv_reports(reports: Mapping[str, Mapping[str, Any]],
                             backends: Iterable[str] | None = None,
                             *, require_exact: bool = True) -> dict[str, Any]:
    """Compare generation reports keyed by backend name.

    ``backends`` (default: every known backend present in ``reports``)
    must name exactly the reports given and include ``pytorch``, whose
    tokens every other backend must reproduce and whose latency the
    speedups divide.  With ``require_exact`` a token difference raises
    ValueError ("token mismatch for backend ...", with the first diverging
    token of each case); otherwise it is reported under ``divergences``."""
    names = list(backends) if backends is not None else [b for b in BACKEND_NAMES if b in reports]
    unknown = sorted(set(names) - set(BACKEND_NAMES))
    if unknown:
        raise ValueError(f"unknown backends: {', '.join(unknown)} "
                         f"(known: {', '.join(BACKEND_NAMES)})")
    if ORACLE_BACKEND not in names:
        raise ValueError(f"the comparison needs a {ORACLE_BACKEND} report (the token oracle)")
    if set(names) != set(reports):
        raise ValueError(f"reports given for {sorted(reports)} but compared backends are {names}")
    problems = [p for b in names for p in _problems_of(b, reports[b])]
    if problems:
        raise ValueError("invalid report: " + "; ".join(problems))
    runs = {b: parse_run(b, reports[b]) for b in names}
    oracle = runs[ORACLE_BACKEND]
    divergences = {b: d for b in names if b != ORACLE_BACKEND
                   for d in [_divergences(oracle, runs[b])] if d}
    if divergences and require_exact:
        raise ValueError("; ".join(_describe(b, d) for b, d in divergences.items()))
    summary = {b: _aggregate(runs[b]) for b in names}
    base = summary[ORACLE_BACKEND]["total_latency_sec"]
    for values in summary.values():
        own = values["total_latency_sec"]
        values["speedup_vs_pytorch"] = base / own if own > 0 else None
    return {
        "schema_version": SCHEMA,
        "tokens_exact": not divergences,
        "token_oracle": ORACLE_BACKEND,
        "case_names": list(oracle.cases),
        "divergences": divergences,
        "backends": summary,
    }


def render_paged_kv_e2e_markdown(result: Mapping[str, Any]) -> str:
    """A Markdown summary: one row per backend, then the first diverging
    token of every case that forked."""
    exact = "yes" if result["tokens_exact"] else "NO"
    out = [f"## Paged-KV backends, end to end ({len(result['case_names'])} cases)", "",
           f"Greedy tokens identical to `{result.get('token_oracle', ORACLE_BACKEND)}` "
           f"on every case: **{exact}**", "",
           "| backend | stage | cases | total s | output tok/s | case p50 s | case p95 s | "
           "case p99 s | peak GiB | speedup |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for name, v in result["backends"].items():
        spread = v["case_latency_sec"]
        speed = "—" if v["speedup_vs_pytorch"] is None else f"{v['speedup_vs_pytorch']:.2f}x"
        out.append(f"| {name} | {v.get('stage', '')} | {v['case_count']} | "
                   f"{v['total_latency_sec']:.4f} | {v['output_tokens_per_sec']:.1f} | "
                   f"{spread['p50_sec']:.4f} | {spread['p95_sec']:.4f} | {spread['p99_sec']:.4f} | "
                   f"{v['peak_gpu_memory_bytes'] / 2**30:.2f} | {speed} |")
    for backend, cases in result.get("divergences", {}).items():
        out += ["", f"### {backend}: cases that diverge", "",
                "| case | first differing token | pytorch | backend | lengths |",
                "|---|---:|---:|---:|---|"]
        for case, d in cases.items():
            if "missing_in" in d:
                out.append(f"| {case} | — | — | — | missing in {d['missing_in']} |")
            else:
                out.append(f"| {case} | {d['index']} | {d['expected']} | {d['got']} | "
                           f"{d['expected_length']} vs {d['got_length']} |")
    return "\n".join(out) + "\n"


def _write_atomically(path: Path, text: str) -> None:
    path.parent.mkdir(parents=True, exist_ok=True)
    staged = path.with_name(f".{path.name}.{os.getpid()}.part")
    staged.write_text(text, encoding="utf-8")
    os.replace(staged, path)


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(
        prog="python -m nanokv.e2e",
        description="Compare greedy tokens, latency, throughput and peak memory of generation "
                    "reports across paged-KV backends (pytorch is the token oracle).")
    for name in BACKEND_NAMES:
        parser.add_argument(f"--{name}", type=Path, metavar="REPORT",
                            help=f"generation report of the {name} backend")
    parser.add_argument("--report", action="append", default=[], metavar="BACKEND=PATH",
                        help="a report given as backend=path (repeatable)")
    parser.add_argument("--output-dir", type=Path, default=Path("paged-kv-e2e-comparison"))
    parser.add_argument("--allow-divergence", action="store_true",
                        help="write the comparison even when tokens differ (exit status 1)")
    return parser


def _report_paths(args: argparse.Namespace) -> dict[str, Path]:
    paths = {name: getattr(args, name) for name in BACKEND_NAMES if getattr(args, name)}
    for item in args.report:
        name, sep, path = item.partition("=")
        if not sep or not name or not path:
            raise SystemExit(f"--report expects BACKEND=PATH, got {item!r}")
        if name in paths:
            raise SystemExit(f"two reports given for backend {name}")
        paths[name] = Path(path)
    if ORACLE_BACKEND not in paths or len(paths) < 2:
        raise SystemExit("give a pytorch report and at least one other backend's report")
    return paths


def main(argv: list[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    reports = {name: json.loads(path.read_text(encoding="utf-8"))
               for name, path in _report_paths(args).items()}
    result = compare_paged_kv_reports(reports, list(reports),
                                      require_exact=not args.allow_divergence)
    markdown = render_paged_kv_e2e_markdown(result)
    _write_atomically(args.output_dir / "paged-kv-e2e-comparison.json",
                      json.dumps(result, indent=2) + "\n")
    _write_atomically(args.output_dir / "paged-kv-e2e-comparison.md", markdown)
    print(markdown, end="")
    return 0 if result["tokens_exact"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
