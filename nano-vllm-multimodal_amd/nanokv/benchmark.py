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
