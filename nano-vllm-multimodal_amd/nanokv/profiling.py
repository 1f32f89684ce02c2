"""rocprofv3 harness: the commands that profile one benchmark case, and the
parser that turns their CSV output into the summaries kept under
``profiles/``.

It plays the part of the reference's Nsight Compute wrapper
(nanovllm/benchmark/ncu.py:22-62 builds the collection command, :86-150
parses and analyses the CSV; scripts/profile_paged_kv_ncu.py:61-142 runs one
case and writes the evidence), for rocprofv3 on MI355X:

* ``trace_command`` / ``counter_command`` build the argument lists.  The
  program always follows ``--`` directly (``python3 bench.py --case C
  --profile-replay N``), and a counter pass holds one counter and runs
  under ``timeout -s KILL``, as rocprofv3 needs a pass of its own per
  counter group.
* ``read_kernel_trace`` / ``read_counters`` parse ``*_kernel_trace.csv`` and
  ``*_counter_collection.csv``; ``kernel_durations`` groups dispatches by
  short kernel name (median, mean, percentiles), ``counter_means`` averages
  a counter per dispatch.
* ``copy_factor`` scales FETCH_SIZE / WRITE_SIZE by what they read for the
  runtime's own device copy of a known size (``bench.py
  --copy-calibration-mib``).
* ``summarize`` / ``render_markdown`` produce the JSON and Markdown that go
  under ``profiles/``.

Command line (on a GPU host; every step is a child process, this module
never touches the GPU itself)::

    python -m nanokv.profiling collect --case chunked_prefill --out DIR
    python -m nanokv.profiling report --case chunked_prefill --out DIR \\
        --profiles profiles
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import re
import statistics
import subprocess
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Iterable, Sequence

HBM_PEAK_GBPS = 8000.0
CASES = ("decode_store", "chunked_prefill", "prefix_gather", "narrow_rows", "decode_step",
         "decode_attention", "grouped_decode_2x8", "grouped_decode_4x7", "grouped_decode_8x4",
         "prefill_attention", "block_pool", "store_floor")
# Cases whose replay launches one kernel in consecutive phases: that
# kernel's dispatches are split evenly among the labels by dispatch order.
PHASES = {"store_floor": {"store_rows_kernel": ("contiguous slots", "chunked-prefill slots")}}
# Runtime kernels a case reports beside its own (the kernel torch's copy_
# runs for a device-to-device copy).  Only their dispatches of the most
# frequent grid are kept: the replay's own launches, not the runtime's
# setup copies of other sizes.
EXTRA_KERNELS = {"store_floor": ("__amd_rocclr_copyBuffer",)}


def modal_grid_only(dispatches: Sequence[Dispatch], prefixes: Sequence[str]) -> list[Dispatch]:
    """Drop the dispatches of kernels named by ``prefixes`` whose grid is not
    the kernel's most frequent grid."""
    keep = _modal_grids([(d.kernel, d.grid) for d in dispatches], prefixes)
    return [d for d in dispatches if not d.kernel.startswith(tuple(prefixes))
            or keep.get(d.kernel) == d.grid]


def _modal_grids(pairs, prefixes) -> dict:
    counts: dict = {}
    for kernel, grid in pairs:
        if kernel.startswith(tuple(prefixes)):
            counts.setdefault(kernel, {}).setdefault(grid, 0)
            counts[kernel][grid] += 1
    return {k: max(v.items(), key=lambda kv: kv[1])[0] for k, v in counts.items()}
GROUPED = {"grouped_decode_2x8": (2, 8), "grouped_decode_4x7": (4, 7), "grouped_decode_8x4": (8, 4)}
MFMA_BF16_PEAK_TFLOPS = 2500.0
COPY_CALIBRATION_MIB = 1024
COPY_KERNEL = "__amd_rocclr_copyBuffer"


# ------------------------------------------------------------------ commands

def trace_command(case: str, out_dir: str | Path, *, replay: int = 20, stem: str = "trace",
                  python: str = "python3", bench: str = "bench.py",
                  rocprof: str = "rocprofv3", settle_s: float | None = None) -> list[str]:
    """Kernel trace + per-kernel stats of ``replay`` replays of one case
    (``settle_s``: the decode-step cases' idle seconds before the replays)."""
    _check_case(case, replay)
    settle = [] if settle_s is None else ["--settle-s", f"{settle_s:g}"]
    return [rocprof, "--kernel-trace", "--stats", "--output-format", "csv", "-d", str(out_dir),
            "-o", stem, "--", python, bench, "--case", case, "--profile-replay", str(replay), *settle]


def counter_command(case: str | None, counter: str, out_dir: str | Path, *, replay: int = 3,
                    stem: str = "pmc", python: str = "python3", bench: str = "bench.py",
                    rocprof: str = "rocprofv3", kill_after_s: int = 120) -> list[str]:
    """One counter pass (FETCH_SIZE or WRITE_SIZE) over ``replay`` replays
    of a case, or over the copy calibration when ``case`` is None."""
    if counter not in ("FETCH_SIZE", "WRITE_SIZE"):
        raise ValueError("one counter per pass: FETCH_SIZE or WRITE_SIZE")
    if case is None:
        program = [python, bench, "--copy-calibration-mib", str(COPY_CALIBRATION_MIB)]
    else:
        _check_case(case, replay)
        program = [python, bench, "--case", case, "--profile-replay", str(replay)]
    return ["timeout", "-s", "KILL", str(kill_after_s), rocprof, "--pmc", counter,
            "--output-format", "csv", "-d", str(out_dir), "-o", stem, "--", *program]


def _check_case(case: str, replay: int) -> None:
    if case not in CASES:
        raise ValueError(f"unknown case {case!r}; one of {', '.join(CASES)}")
    if replay <= 0:
        raise ValueError("replay count must be positive")


def collection_plan(case: str, out: Path, *, replay: int = 20, counter_replay: int = 3,
                    python: str = "python3") -> list[tuple[str, list[str]]]:
    """The five passes behind one case's summary: the trace, the case's
    FETCH_SIZE and WRITE_SIZE, and the same two counters on the copy."""
    return [
        ("trace", trace_command(case, out / "trace", replay=replay, python=python)),
        ("fetch", counter_command(case, "FETCH_SIZE", out / "fetch", replay=counter_replay,
                                  python=python)),
        ("write", counter_command(case, "WRITE_SIZE", out / "write", replay=counter_replay,
                                  python=python)),
        ("copy_fetch", counter_command(None, "FETCH_SIZE", out / "copy_fetch", python=python)),
        ("copy_write", counter_command(None, "WRITE_SIZE", out / "copy_write", python=python)),
    ]


def trace_kernel_here(case: str, kernel_prefix: str, *, replay: int = 10, timeout_s: int = 300,
                      bench: str | Path | None = None, settle_s: float | None = None,
                      echo: bool = False) -> dict:
    """Run ``trace_command(case)`` as a child process on this host (in a
    scratch directory under /tmp, TMPDIR=/tmp, the program straight after
    ``--``) and return the trace statistics of the first kernel whose short
    name starts with ``kernel_prefix`` (warmup dispatch skipped), with the
    command.  Never raises: a missing profiler, a time-out or output without
    that kernel gives ``{"error": ...}``.  rocprofv3 may exit non-zero after
    the program finished and wrote its trace; the trace is used whenever the
    replay printed its last line.  ``echo`` forwards the child's output to
    stderr line by line as it arrives."""
    import shutil
    import signal
    import tempfile
    import threading

    rocprof = shutil.which("rocprofv3") or ("/opt/rocm/bin/rocprofv3"
                                             if os.path.exists("/opt/rocm/bin/rocprofv3") else None)
    if rocprof is None:
        return {"error": "rocprofv3 not found"}
    bench_path = str(Path(bench) if bench else Path(__file__).resolve().parents[2] / "bench.py")
    scratch = tempfile.mkdtemp(prefix="nanokv_trace_", dir="/tmp")
    try:
        command = trace_command(case, Path(scratch) / "trace", replay=replay, python=sys.executable,
                                bench=bench_path, rocprof=rocprof, settle_s=settle_s)
        env = dict(os.environ, TMPDIR="/tmp")
        proc = subprocess.Popen(command, cwd="/tmp", env=env, stdout=subprocess.PIPE,
                                stderr=subprocess.STDOUT, text=True, start_new_session=True)
        lines: list[str] = []

        def forward() -> None:  # the child's lines as they come, so a slow start shows
            for line in proc.stdout:
                lines.append(line)
                if echo:
                    print(f"[trace] {line.rstrip()}", file=sys.stderr, flush=True)

        reader = threading.Thread(target=forward, daemon=True)
        reader.start()
        try:
            proc.wait(timeout=timeout_s)
        except subprocess.TimeoutExpired:
            os.killpg(proc.pid, signal.SIGKILL)
            proc.wait()
            reader.join(timeout=10)
            return {"error": f"trace of {case} did not finish in {timeout_s} s"}
        reader.join(timeout=10)
        output = "".join(lines)
        if "profile replay complete" not in output:
            tail = output.strip().splitlines()[-3:]
            return {"error": f"replay of {case} did not complete (exit {proc.returncode}): "
                             + " | ".join(tail)}
        try:
            trace = kernel_durations(read_kernel_trace(_find_csv(Path(scratch) / "trace",
                                                                 "_kernel_trace.csv")),
                                     skip_first=1)
        except (OSError, ValueError, KeyError) as exc:
            return {"error": f"no kernel trace: {exc}"}
        name = next((k for k in trace if k.startswith(kernel_prefix)), None)
        if name is None:
            return {"error": f"no {kernel_prefix}* dispatch in the trace"}
        return {"kernel": name, **trace[name], "rocprof_exit": proc.returncode,
                "command": " ".join([os.path.basename(rocprof), *command[1:]])}
    finally:
        shutil.rmtree(scratch, ignore_errors=True)


# ------------------------------------------------------------------- parsing

def short_name(kernel: str) -> str:
    """``void nkv::(anonymous namespace)::store_rows_kernel<16>(unsigned
    char const*, ...)`` -> ``store_rows_kernel<16>``: the name without
    return type, namespaces and parameter list (template arguments kept)."""
    text = kernel.strip()
    depth, cut = 0, len(text)
    for i, ch in enumerate(text):  # the parameter list is the first '(' at depth 0
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and not text.startswith("(anonymous", i):
            cut = i
            break
    head = text[:cut]
    head = re.sub(r"^void\s+", "", head)
    head = head.replace("(anonymous namespace)::", "")
    # drop the namespaces before the last '::' outside template brackets
    depth, last = 0, -1
    for i in range(len(head) - 1):
        if head[i] == "<":
            depth += 1
        elif head[i] == ">":
            depth -= 1
        elif head[i:i + 2] == "::" and depth == 0:
            last = i + 2
    return head[last:] if last >= 0 else head


@dataclass(frozen=True)
class Dispatch:
    kernel: str        # short name
    dispatch_id: int
    start_ns: int
    end_ns: int
    grid: tuple[int, int, int]
    workgroup: tuple[int, int, int]

    @property
    def duration_ns(self) -> int:
        return self.end_ns - self.start_ns


def read_kernel_trace(path: str | Path) -> list[Dispatch]:
    """Every dispatch of a ``*_kernel_trace.csv``, in dispatch order."""
    out = []
    with open(path, newline="") as handle:
        for row in csv.DictReader(handle):
            out.append(Dispatch(
                kernel=short_name(row["Kernel_Name"]),
                dispatch_id=int(row["Dispatch_Id"]),
                start_ns=int(row["Start_Timestamp"]),
                end_ns=int(row["End_Timestamp"]),
                grid=tuple(int(row[f"Grid_Size_{a}"]) for a in "XYZ"),
                workgroup=tuple(int(row[f"Workgroup_Size_{a}"]) for a in "XYZ"),
            ))
    out.sort(key=lambda d: d.dispatch_id)
    return out


def label_phases(dispatches: Sequence[Dispatch], phases: dict[str, Sequence[str]]) -> list[Dispatch]:
    """Rename the dispatches of each kernel named in ``phases`` (by short-name
    prefix) to ``"<name> [<label>]"``, the labels taken in dispatch order,
    an equal share of the dispatches each."""
    out = list(dispatches)
    for prefix, labels in phases.items():
        picked = [i for i, d in enumerate(out) if d.kernel.startswith(prefix)]
        per = max(1, len(picked) // len(labels))
        for j, i in enumerate(picked):
            label = labels[min(j // per, len(labels) - 1)]
            d = out[i]
            out[i] = Dispatch(f"{d.kernel} [{label}]", d.dispatch_id, d.start_ns, d.end_ns, d.grid,
                              d.workgroup)
    return out


def label_counter_phases(rows: Sequence[dict], phases: dict[str, Sequence[str]]) -> list[dict]:
    """:func:`label_phases` for counter rows (one or more rows per dispatch)."""
    out = [dict(r) for r in rows]
    for prefix, labels in phases.items():
        ids = sorted({r["dispatch_id"] for r in out if r["kernel"].startswith(prefix)})
        per = max(1, len(ids) // len(labels))
        rank = {d: labels[min(j // per, len(labels) - 1)] for j, d in enumerate(ids)}
        for r in out:
            if r["dispatch_id"] in rank and r["kernel"].startswith(prefix):
                r["kernel"] = f"{r['kernel']} [{rank[r['dispatch_id']]}]"
    return out


def _percentile(sorted_values: Sequence[float], q: float) -> float:
    position = (len(sorted_values) - 1) * q
    lo = int(position)
    hi = min(lo + 1, len(sorted_values) - 1)
    return sorted_values[lo] + (sorted_values[hi] - sorted_values[lo]) * (position - lo)


def kernel_durations(dispatches: Iterable[Dispatch], *, skip_first: int = 0) -> dict[str, dict]:
    """Per short kernel name: dispatch count and duration statistics in µs
    (median, mean, min, max, p05, p95), skipping each kernel's first
    ``skip_first`` dispatches (warmup)."""
    by_kernel: dict[str, list[float]] = {}
    seen: dict[str, int] = {}
    for d in dispatches:
        seen[d.kernel] = seen.get(d.kernel, 0) + 1
        if seen[d.kernel] > skip_first:
            by_kernel.setdefault(d.kernel, []).append(d.duration_ns / 1e3)
    stats = {}
    for name, values in by_kernel.items():
        ordered = sorted(values)
        stats[name] = {
            "dispatches": len(values),
            "median_us": statistics.median(ordered),
            "mean_us": statistics.fmean(ordered),
            "min_us": ordered[0],
            "max_us": ordered[-1],
            "p05_us": _percentile(ordered, 0.05),
            "p95_us": _percentile(ordered, 0.95),
        }
    return stats


def read_counters(path: str | Path) -> list[dict]:
    """Rows of a ``*_counter_collection.csv``: kernel (short name),
    dispatch id, counter name and value."""
    out = []
    with open(path, newline="") as handle:
        for row in csv.DictReader(handle):
            out.append({"kernel": short_name(row["Kernel_Name"]),
                        "dispatch_id": int(row["Dispatch_Id"]),
                        "grid": int(row.get("Grid_Size") or 0),
                        "counter": row["Counter_Name"].strip(),
                        "value": float(row["Counter_Value"])})
    return out


def counter_means(rows: Iterable[dict], counter: str) -> dict[str, dict]:
    """Per kernel: the counter summed over each dispatch's rows (a counter
    may come per XCD or per instance), then averaged over dispatches."""
    per_dispatch: dict[tuple[str, int], float] = {}
    for r in rows:
        if r["counter"] == counter:
            key = (r["kernel"], r["dispatch_id"])
            per_dispatch[key] = per_dispatch.get(key, 0.0) + r["value"]
    grouped: dict[str, list[float]] = {}
    for (kernel, _), value in per_dispatch.items():
        grouped.setdefault(kernel, []).append(value)
    return {k: {"dispatches": len(v), "mean": statistics.fmean(v), "min": min(v), "max": max(v)}
            for k, v in grouped.items()}


def copy_factor(rows: Iterable[dict], counter: str,
                bytes_per_copy: int = COPY_CALIBRATION_MIB << 20) -> float:
    """Counter reading per true byte for the runtime's copy kernel, which
    reads and writes ``bytes_per_copy`` bytes per launch (FETCH_SIZE and
    WRITE_SIZE count KiB)."""
    means = counter_means(rows, counter)
    copies = [v for k, v in means.items() if k.startswith(COPY_KERNEL)]
    if not copies:
        raise ValueError(f"no {COPY_KERNEL} dispatch in the calibration counters")
    return copies[0]["mean"] * 1024.0 / bytes_per_copy


# ------------------------------------------------------------------- summary

def _find_csv(directory: Path, suffix: str) -> Path:
    found = sorted(Path(directory).rglob(f"*{suffix}"))
    if not found:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    return found[0]


def summarize(case: str, out: Path, algorithmic_bytes: dict[str, int], *,
              commands: dict[str, list[str]] | None = None, skip_first: int = 1,
              algorithmic_flops: dict[str, int] | None = None) -> dict:
    """One case's figures from the five passes under ``out``: per kernel the
    trace statistics, the achieved bandwidth on its median duration
    (algorithmic bytes per launch from ``algorithmic_bytes``, keyed by a
    prefix of the short kernel name) and the calibrated HBM traffic."""
    phases = PHASES.get(case, {})
    extra = EXTRA_KERNELS.get(case, ())
    trace = kernel_durations(
        label_phases(modal_grid_only(read_kernel_trace(_find_csv(out / "trace", "_kernel_trace.csv")),
                                     extra), phases),
        skip_first=skip_first)
    factors, traffic = {}, {}
    for counter, key in (("FETCH_SIZE", "fetch"), ("WRITE_SIZE", "write")):
        copy_dir, case_dir = out / f"copy_{key}", out / key
        if copy_dir.is_dir() and case_dir.is_dir():
            factors[counter] = copy_factor(read_counters(_find_csv(copy_dir, "_counter_collection.csv")),
                                           counter)
            rows = read_counters(_find_csv(case_dir, "_counter_collection.csv"))
            keep = _modal_grids([(r["kernel"], r["grid"]) for r in rows], extra)
            rows = [r for r in rows if not r["kernel"].startswith(tuple(extra))
                    or keep.get(r["kernel"]) == r["grid"]]
            traffic[counter] = counter_means(label_counter_phases(rows, phases), counter)
    reported = ("nkv", "store_", "gather_", "build_", "pack_", "attn_", "pool_", *extra)
    kernels = {}
    for name, stats in sorted(trace.items(), key=lambda kv: -kv[1]["median_us"] * kv[1]["dispatches"]):
        if not name.startswith(reported):
            continue
        record = dict(stats)
        nbytes = next((b for prefix, b in algorithmic_bytes.items() if name.startswith(prefix)), None)
        if nbytes:
            record["algorithmic_bytes"] = nbytes
            record["achieved_gbps_at_median"] = nbytes / (stats["median_us"] * 1e3)
            record["hbm_fraction_at_median"] = record["achieved_gbps_at_median"] / HBM_PEAK_GBPS
        flops = next((f for prefix, f in (algorithmic_flops or {}).items() if name.startswith(prefix)),
                     None)
        if flops:
            record["algorithmic_flops"] = flops
            record["achieved_tflops_at_median"] = flops / (stats["median_us"] * 1e6)
            record["mfma_fraction_at_median"] = record["achieved_tflops_at_median"] / MFMA_BF16_PEAK_TFLOPS
        moved = {}
        for counter, per_kernel in traffic.items():
            if name in per_kernel:
                moved[counter] = per_kernel[name]["mean"] * 1024.0 / factors[counter]
        if len(moved) == 2:
            record["hbm_read_bytes"] = round(moved["FETCH_SIZE"])
            record["hbm_write_bytes"] = round(moved["WRITE_SIZE"])
            record["traffic_bytes"] = round(moved["FETCH_SIZE"] + moved["WRITE_SIZE"])
            if nbytes:
                record["traffic_over_algorithmic"] = record["traffic_bytes"] / nbytes
            # the rate in bytes that actually crossed the HBM interface
            record["hbm_gbps_at_median"] = record["traffic_bytes"] / (stats["median_us"] * 1e3)
        kernels[name] = record
    return {
        "schema_version": "nanokv.rocprof_summary.v1",
        "case": case,
        "peak_gbps": HBM_PEAK_GBPS,
        "counter_factors": factors,
        "warmup_dispatches_skipped": skip_first,
        "kernels": kernels,
        "commands": {k: " ".join(v) for k, v in (commands or {}).items()},
    }


def render_markdown(summary: dict, title: str | None = None) -> str:
    lines = [f"# rocprofv3 summary: {title or summary['case']} (MI355X)", "",
             "Written by `python -m nanokv.profiling report` from the CSVs of the passes below "
             "(run from the repository root on the GPU host, `TMPDIR=/tmp`):", "", "```"]
    lines += list(summary["commands"].values()) or ["(commands not recorded)"]
    lines += ["```", "",
              f"Durations are per dispatch from the kernel trace, each kernel's first "
              f"{summary['warmup_dispatches_skipped']} dispatch(es) skipped. Bandwidth is the "
              f"kernel's algorithmic bytes per launch over its median duration, against "
              f"{summary['peak_gbps'] / 1000:.1f} TB/s.", "",
              "| Kernel | Dispatches | Median (µs) | Mean (µs) | p05–p95 (µs) | Algorithmic bytes "
              "| GB/s at median | % of peak |",
              "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for name, k in summary["kernels"].items():
        gbps = k.get("achieved_gbps_at_median")
        lines.append(
            f"| `{name}` | {k['dispatches']} | {k['median_us']:.2f} | {k['mean_us']:.2f} | "
            f"{k['p05_us']:.2f}–{k['p95_us']:.2f} | "
            + (f"{k['algorithmic_bytes']:,} | {gbps:,.0f} | {100 * gbps / summary['peak_gbps']:.1f}% |"
               if gbps else "— | — | — |"))
    mfma = {n: k for n, k in summary["kernels"].items() if "achieved_tflops_at_median" in k}
    if mfma:
        lines += ["", f"MFMA-bound kernels against the dense bf16 peak of {MFMA_BF16_PEAK_TFLOPS:,.0f} "
                      "TFLOP/s:", "", "| Kernel | Algorithmic FLOPs | TFLOP/s at median | % of peak |",
                  "|---|---:|---:|---:|"]
        for name, k in mfma.items():
            lines.append(f"| `{name}` | {k['algorithmic_flops']:,} | {k['achieved_tflops_at_median']:.1f} | "
                         f"{100 * k['mfma_fraction_at_median']:.1f}% |")
    if summary["counter_factors"]:
        f = summary["counter_factors"]
        lines += ["", "## HBM traffic (FETCH_SIZE / WRITE_SIZE)", "",
                  f"Scaled by the counters' reading for the runtime's copy of "
                  f"{COPY_CALIBRATION_MIB} MiB (`{COPY_KERNEL}`): FETCH_SIZE reads "
                  f"{f.get('FETCH_SIZE', float('nan')):.4f}x and WRITE_SIZE "
                  f"{f.get('WRITE_SIZE', float('nan')):.4f}x the true bytes.", "",
                  "The last two columns are the rate in counter bytes (what crossed the HBM "
                  "interface) over the median duration, and its fraction of peak.", "",
                  "| Kernel | HBM read (B) | HBM written (B) | Total (B) | Algorithmic (B) | Ratio "
                  "| HBM GB/s at median | % of peak |",
                  "|---|---:|---:|---:|---:|---:|---:|---:|"]
        for name, k in summary["kernels"].items():
            if "traffic_bytes" in k:
                alg = k.get("algorithmic_bytes")
                hbm = k["traffic_bytes"] / (k["median_us"] * 1e3)
                lines.append(f"| `{name}` | {k['hbm_read_bytes']:,} | {k['hbm_write_bytes']:,} | "
                             f"{k['traffic_bytes']:,} | " + (f"{alg:,} | {k['traffic_over_algorithmic']:.3f} |"
                                                              if alg else "— | — |")
                             + f" {hbm:,.0f} | {100 * hbm / summary['peak_gbps']:.1f}% |")
    return "\n".join(lines) + "\n"


def algorithmic_flops_for(case: str) -> dict[str, int]:
    """Algorithmic FLOPs per launch of the case's MFMA-bound kernels: the
    chunked-prefill step's causal attention, 4 x head_dim x query heads x
    the (query, visible key) pairs of 16 requests (query lengths scaled to
    8,192 tokens, 8 continuing after 1-4 cached 256-row blocks, seed 17)."""
    if case != "prefill_attention":
        return {}
    import numpy as np

    rng = np.random.default_rng(17)
    raw = rng.integers(128, 4097, 16).astype(np.float64)
    q_lens = np.floor(raw / raw.sum() * 8192).astype(np.int64)
    q_lens[-1] += 8192 - q_lens.sum()
    cached = np.zeros(16, np.int64)
    cached[:8] = rng.integers(1, 5, 8) * 256
    pairs = int(sum(lq * (lq + 1) // 2 + lq * c for lq, c in zip(q_lens.tolist(), cached.tolist())))
    return {"attn_prefill_kernel": 4 * 128 * 16 * pairs}


def algorithmic_bytes_for(case: str) -> dict[str, int]:
    """Algorithmic bytes per launch of the case's kernels (the workload's
    own byte counts), keyed by short-name prefix."""
    from nanokv import workloads

    if case == "decode_attention":
        wl = workloads.build("decode_step", num_layers=1)
        total = int(wl.num_tokens.sum())
        q_bytes = wl.num_seqs * 16 * wl.head_dim * 2
        nbytes = total * wl.row_bytes * 2 + 2 * q_bytes
        # the entry split at 8 kv heads, the range split below
        return {"attn_decode_entry_kernel": nbytes, "attn_decode_range_kernel": nbytes}
    if case in GROUPED:
        hkv, group = GROUPED[case]
        wl = workloads.build("decode_step", num_layers=1)
        total = int(wl.num_tokens.sum())
        q_bytes = wl.num_seqs * hkv * group * 128 * 2
        nbytes = total * hkv * 128 * 2 * 2 + 2 * q_bytes
        return {"attn_decode_entry_kernel": nbytes, "attn_decode_range_kernel": nbytes}
    if case in ("prefill_attention", "block_pool"):
        return {}
    if case == "store_floor":
        wl = workloads.build("chunked_prefill")
        return {"__amd_rocclr_copyBuffer": 67_108_864, "store_rows_kernel": wl.store_bytes(layers=1)}
    wl = workloads.build(case, num_layers=1) if case == "decode_step" else workloads.build(case)
    found = {}
    if wl.slot_mapping is not None:
        found["store_rows_kernel"] = wl.store_bytes(layers=1)
    if case != "decode_store":
        found["gather_planned_kernel"] = wl.gather_bytes(layers=1)
    if case in ("chunked_prefill", "narrow_rows"):
        found["store_gather_kernel"] = wl.store_gather_bytes(layers=1)
    return found


# ---------------------------------------------------------------- command line

def main(argv: Sequence[str] | None = None) -> int:
    parser = argparse.ArgumentParser(prog="python -m nanokv.profiling", description=__doc__,
                                     formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("action", choices=("collect", "report", "commands"))
    parser.add_argument("--case", required=True, choices=CASES)
    parser.add_argument("--out", type=Path, required=True, help="directory of the raw passes")
    parser.add_argument("--profiles", type=Path, default=Path("profiles"))
    parser.add_argument("--replay", type=int, default=20)
    parser.add_argument("--counter-replay", type=int, default=3)
    parser.add_argument("--python", default="python3")
    parser.add_argument("--name", help="file stem under --profiles (default: <case>_rocprof)")
    args = parser.parse_args(argv)
    plan = collection_plan(args.case, args.out, replay=args.replay,
                           counter_replay=args.counter_replay, python=args.python)
    if args.action == "commands":
        for _, command in plan:
            print(" ".join(command))
        return 0
    if args.action == "collect":
        env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
        for label, command in plan:
            print(f"[profiling] {label}: {' '.join(command)}", flush=True)
            done = subprocess.run(command, env=env)
            if done.returncode != 0:
                print(f"[profiling] {label} failed with status {done.returncode}", flush=True)
                return done.returncode
        (args.out / "commands.json").write_text(json.dumps({k: v for k, v in plan}, indent=1))
        return 0
    recorded = args.out / "commands.json"
    commands = json.loads(recorded.read_text()) if recorded.is_file() else dict(plan)
    summary = summarize(args.case, args.out, algorithmic_bytes_for(args.case), commands=commands,
                        algorithmic_flops=algorithmic_flops_for(args.case))
    stem = args.name or f"{args.case}_rocprof"
    args.profiles.mkdir(parents=True, exist_ok=True)
    (args.profiles / f"{stem}.json").write_text(json.dumps(summary, indent=1) + "\n")
    (args.profiles / f"{stem}.md").write_text(render_markdown(summary))
    print(render_markdown(summary))
    return 0


if __name__ == "__main__":
    sys.exit(main())
