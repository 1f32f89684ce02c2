"""Measurement helpers: latency percentiles, HBM roofline constants and
per-launch event timing.

``linear_percentile`` and the p50/p95/p99 summary follow the reference's
benchmark (nanovllm/benchmark/metrics.py:82-92,
nanovllm/benchmark/paged_kv.py:202-214); ``effective_bytes`` is the
reference's payload count (paged_kv.py:196-199), reported next to the
algorithmic byte counts of nanokv.workloads.Workload.
"""
from __future__ import annotations

from statistics import fmean
from typing import Iterable, Sequence

import torch

MI355X_HBM_PEAK_GBPS = 8000.0  # 8 TB/s HBM3E, decimal GB


def linear_percentile(values: Sequence[float], quantile: float) -> float:
    if not values:
        raise ValueError("percentile requires at least one value")
    if not 0.0 <= quantile <= 1.0:
        raise ValueError("quantile must be between zero and one")
    ordered = sorted(values)
    position = (len(ordered) - 1) * quantile
    lower = int(position)
    upper = min(lower + 1, len(ordered) - 1)
    return ordered[lower] + (ordered[upper] - ordered[lower]) * (position - lower)


def summarize_latencies(samples_us: Iterable[float]) -> dict[str, float]:
    samples = tuple(float(v) for v in samples_us)
    if not samples or any(v < 0 for v in samples):
        raise ValueError("latency samples must be non-empty and non-negative")
    return {
        "count": len(samples),
        "mean_us": fmean(samples),
        "min_us": min(samples),
        "max_us": max(samples),
        "p50_us": linear_percentile(samples, 0.50),
        "p95_us": linear_percentile(samples, 0.95),
        "p99_us": linear_percentile(samples, 0.99),
    }


def effective_bytes(operation: str, num_tokens: int, num_kv_heads: int, head_dim: int,
                    element_size: int) -> int:
    payload = num_tokens * num_kv_heads * head_dim * element_size
    return payload * (4 if operation == "store" else 2)


class LaunchTimer:
    """Brackets individual launches with events recorded on the stream the
    kernels run on (the tensors' current stream), and reports the mean
    duration of the bracketed launches in microseconds."""

    def __init__(self, stream: torch.cuda.Stream) -> None:
        self.stream = stream
        self.pairs: list[tuple[torch.cuda.Event, torch.cuda.Event]] = []

    def start(self) -> torch.cuda.Event:
        event = torch.cuda.Event(enable_timing=True)
        event.record(self.stream)
        return event

    def stop(self, start: torch.cuda.Event) -> None:
        event = torch.cuda.Event(enable_timing=True)
        event.record(self.stream)
        self.pairs.append((start, event))

    def durations_us(self) -> list[float]:
        if self.pairs:
            self.pairs[-1][1].synchronize()
        return [a.elapsed_time(b) * 1000.0 for a, b in self.pairs]

    def mean_us(self) -> float:
        values = self.durations_us()
        return fmean(values) if values else 0.0


# ------------------------------------------------------------- workloads CLI

FLUSH_BYTES = 512 << 20  # > the 256 MB MALL


def _time_with_flush(fn, flush: torch.Tensor, iterations: int, warmup: int) -> list[float]:
    """Per-iteration event timing of ``fn``; before each timed call a
    512 MiB read (a sum over the flush buffer) evicts the MALL / L2, so
    re-reads cannot be served from on-die caches.  The eviction reads rather
    than writes, so the timed call does not pay for writing back dirty lines
    it did not make.  The read is outside the bracketed region."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    words = flush.view(torch.int64)
    pairs = []
    for _ in range(iterations):
        words.sum()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        fn()
        end.record(stream)
        pairs.append((start, end))
    torch.cuda.synchronize()
    return [a.elapsed_time(b) * 1000.0 for a, b in pairs]


def run_workload(name: str, *, iterations: int = 50, warmup: int = 5, device=None) -> list[dict]:
    """Measure the HIP path on one named workload (nanokv.workloads) and
    return one record per operation: algorithmic bytes, latency summary,
    GB/s at p50 and the fraction of the HBM peak."""
    import numpy as np

    from nanokv import workloads
    from nanokv.packing import DevicePacker, SequenceBatch
    from nanokv.paged_kv import create_paged_kv_backend

    device = device or torch.device("cuda", 0)
    backend = create_paged_kv_backend("hip")
    wl = workloads.build(name) if name != "decode_step" else workloads.build(name, num_layers=1)
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    kc = torch.empty(shape, dtype=wl.dtype, device=device).normal_()
    vc = torch.empty_like(kc).normal_()
    flush = torch.zeros(FLUSH_BYTES, dtype=torch.uint8, device=device)
    element = torch.empty((), dtype=wl.dtype).element_size()
    records = []

    def record(op, nbytes, samples, reference_bytes):
        summary = summarize_latencies(samples)
        gbps = nbytes / (summary["p50_us"] * 1e-6) / 1e9
        records.append({
            "workload": name, "operation": op, "algorithmic_bytes": nbytes,
            "reference_effective_bytes": reference_bytes, "latency": summary,
            "gbps_at_p50": round(gbps, 2), "hbm_fraction": round(gbps / MI355X_HBM_PEAK_GBPS, 4),
        })

    if wl.slot_mapping is not None:
        key = (wl.key[0] if wl.key.ndim == 4 else wl.key).to(device)
        value = (wl.value[0] if wl.value.ndim == 4 else wl.value).to(device)
        slots = torch.from_numpy(wl.slot_mapping).to(device)
        samples = _time_with_flush(lambda: backend.store(key, value, kc, vc, slots), flush,
                                   iterations, warmup)
        record("store", wl.store_bytes(layers=1), samples,
               effective_bytes("store", int(wl.slot_mapping.size), wl.num_kv_heads, wl.head_dim, element))
    if name != "decode_store":
        offsets, ids = wl.csr()
        packer = DevicePacker(device, wl.block_size)
        batch = SequenceBatch(wl.num_tokens, offsets, ids, wl.num_prompt, wl.num_cached, wl.num_scheduled)
        if wl.phase == "decode":
            samples = _time_with_flush(lambda: packer.pack_decode(batch), flush, iterations, warmup)
            record("pack_decode", 0, samples, 0)
        else:
            samples = _time_with_flush(lambda: packer.pack_prefill(batch, force_block_tables=True),
                                       flush, iterations, warmup)
            record("pack_prefill", 0, samples, 0)
        tables = torch.from_numpy(wl.padded_block_tables()).to(device)
        cu = torch.from_numpy(wl.cu_seqlens_k()).to(device)
        total = int(wl.context_lens.astype(np.int64).sum())
        plan = backend.build_gather_plan(kc, tables, cu, total)
        k_out = torch.empty((total, wl.num_kv_heads, wl.head_dim), dtype=wl.dtype, device=device)
        v_out = torch.empty_like(k_out)
        samples = _time_with_flush(
            lambda: backend.gather_varlen(kc, vc, tables, cu, total, plan=plan, out=(k_out, v_out)),
            flush, iterations, warmup)
        record("gather_varlen_kv", wl.gather_bytes(layers=1), samples,
               2 * effective_bytes("gather", total, wl.num_kv_heads, wl.head_dim, element))
        samples = _time_with_flush(lambda: backend.build_gather_plan(kc, tables, cu, total), flush,
                                   iterations, warmup)
        record("build_gather_plan", 0, samples, 0)
    for r in records:
        if r["algorithmic_bytes"] == 0:
            r["gbps_at_p50"] = None
            r["hbm_fraction"] = None
    return records


def render_markdown(records: list[dict]) -> str:
    lines = ["| Workload | Operation | Algorithmic bytes | p50 (us) | p95 (us) | GB/s at p50 | HBM fraction |",
             "|---|---|---:|---:|---:|---:|---:|"]
    for r in records:
        gbps = "—" if r["gbps_at_p50"] is None else f"{r['gbps_at_p50']:.1f}"
        frac = "—" if r["hbm_fraction"] is None else f"{100 * r['hbm_fraction']:.1f}%"
        lines.append(f"| {r['workload']} | {r['operation']} | {r['algorithmic_bytes']:,} | "
                     f"{r['latency']['p50_us']:.2f} | {r['latency']['p95_us']:.2f} | {gbps} | {frac} |")
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    import argparse
    import json

    from nanokv import workloads

    parser = argparse.ArgumentParser(description="Per-workload paged-KV benchmark of the hip backend")
    parser.add_argument("--workloads", default=",".join(workloads.WORKLOAD_NAMES))
    parser.add_argument("--iterations", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--json", help="also write the records to this file")
    args = parser.parse_args(argv)
    records = []
    for name in args.workloads.split(","):
        print(f"[benchmark] {name}", flush=True)
        records.extend(run_workload(name.strip(), iterations=args.iterations, warmup=args.warmup))
        torch.cuda.empty_cache()
    print(render_markdown(records), flush=True)
    if args.json:
        with open(args.json, "w") as handle:
            json.dump({"schema_version": "nanokv.paged_kv_workloads.v1", "records": records}, handle, indent=1)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
