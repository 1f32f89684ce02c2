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


# ------------------------------------------------ the reference's own algorithm

class TorchReferenceBackend:
    """The reference's ``pytorch`` paged-KV backend
    (nanovllm/layers/paged_kv/pytorch_backend.py:26-50) restated with the
    same validators and the same torch ops, for timing the reference's
    algorithm beside the hip backend, on the GPU or on host tensors: the
    store masks out -1 slots (on a GPU a device-to-host sync) and scatters
    with ``index_copy_``; the gather copies whole blocks with
    ``index_select`` and slices them to the length.  Never used by the hip
    backend itself."""

    name = "torch-reference"

    def store(self, key, value, key_cache, value_cache, slot_mapping):
        from nanokv.paged_kv import validate_store_inputs

        validate_store_inputs(key, value, key_cache, value_cache, slot_mapping)
        keep = slot_mapping >= 0
        rows = slot_mapping[keep].to(dtype=torch.long)
        key_cache.flatten(0, 1).index_copy_(0, rows, key[keep])
        value_cache.flatten(0, 1).index_copy_(0, rows, value[keep])

    def gather(self, cache, block_table, sequence_length):
        from nanokv.paged_kv import validate_gather_inputs

        dims = validate_gather_inputs(cache, block_table, sequence_length)
        if dims.required_blocks == 0:
            return cache.new_empty((0, dims.num_kv_heads, dims.head_dim))
        ids = block_table[: dims.required_blocks].to(dtype=torch.long)
        return cache.index_select(0, ids).flatten(0, 1)[:sequence_length]


# -------------------------------------------------------- environment identity

def cpu_model() -> str:
    """The host CPU's model name (``lscpu``, else /proc/cpuinfo)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as handle:
            for line in handle:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads() -> int:
    """Threads a CPU measurement may use: the cores this process may run on,
    capped by OMP_NUM_THREADS when the host sets it (a shared host gives a
    job a share of its cores, whatever os.cpu_count() says)."""
    import os

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(cores, int(cap))) if cap.isdigit() and int(cap) > 0 else max(1, cores)


def environment_identity(device=None) -> dict:
    """Who measured: time, software versions, GPU name / UUID / arch / CU
    count / memory, the HIP status of torch, and the host CPU (the fields of
    the reference's benchmark identity, nanovllm/benchmark/paged_kv.py:
    364-384, with ROCm's own)."""
    import datetime
    import os
    import platform
    import sys

    identity = {
        "timestamp_utc": datetime.datetime.now(datetime.timezone.utc).isoformat(),
        "python": sys.version.split()[0],
        "platform": platform.platform(),
        "torch": torch.__version__,
        "torch_hip": torch.version.hip,
        "hip_status": ("pytorch_rocm_available" if torch.version.hip is not None and torch.cuda.is_available()
                       else "pytorch_rocm_without_gpu" if torch.version.hip is not None
                       else "not_a_rocm_build"),
        "cpu_model": cpu_model(),
        "cpu_count": os.cpu_count(),
        "host_threads": host_threads(),
    }
    try:
        from nanokv import _lib

        identity["nanokv_build_id"] = _lib.build_id()
        identity["nanokv_library"] = _lib.library_path()
    except RuntimeError as exc:  # not built: the identity says so
        identity["nanokv_build_id"] = f"unavailable: {exc}"
    if device is not None and torch.cuda.is_available():
        props = torch.cuda.get_device_properties(device)
        identity.update({
            "device": str(device),
            "gpu_name": props.name,
            "gpu_uuid": str(getattr(props, "uuid", "unavailable")),
            "gpu_arch": getattr(props, "gcnArchName", "unknown"),
            "compute_units": props.multi_processor_count,
            "gpu_memory_bytes": props.total_memory,
        })
    return identity


# ------------------------------------------------------------- workloads

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


class PreparedWorkload:
    """One single-layer workload (nanokv.workloads) resident on a device,
    with its operations as zero-argument calls in step order (``store``,
    then ``gather_varlen_kv`` after the plan is built) and their algorithmic
    and reference-counted bytes.  On the GPU the calls are the hip backend's;
    ``check()`` compares them bit-exactly with the torch restatement of the
    reference backend on the same device."""

    def __init__(self, name: str, device, backend=None):
        import numpy as np

        from nanokv import workloads

        self.name = name
        self.device = torch.device(device)
        wl = workloads.build(name) if name != "decode_step" else workloads.build(name, num_layers=1)
        self.wl = wl
        shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
        gen = torch.Generator(device=self.device).manual_seed(workloads.seed_for(name))
        self.key_cache = torch.empty(shape, dtype=wl.dtype, device=self.device).normal_(generator=gen)
        self.value_cache = torch.empty_like(self.key_cache).normal_(generator=gen)
        element = torch.empty((), dtype=wl.dtype).element_size()
        self.ops: dict = {}
        self.algorithmic_bytes: dict[str, int] = {}
        self.reference_bytes: dict[str, int] = {}
        self.tables = torch.from_numpy(wl.padded_block_tables()).to(self.device)
        self.cu = torch.from_numpy(wl.cu_seqlens_k()).to(self.device)
        self.context_lens = wl.context_lens.astype(np.int64)
        self.total = int(self.context_lens.sum())
        if backend is None:
            from nanokv.paged_kv import create_paged_kv_backend

            backend = create_paged_kv_backend("hip")
        self.backend = backend
        if wl.slot_mapping is not None:
            self.key = (wl.key[0] if wl.key.ndim == 4 else wl.key).to(self.device)
            self.value = (wl.value[0] if wl.value.ndim == 4 else wl.value).to(self.device)
            self.slots = torch.from_numpy(wl.slot_mapping).to(self.device)
            self.ops["store"] = lambda: backend.store(self.key, self.value, self.key_cache,
                                                      self.value_cache, self.slots)
            self.algorithmic_bytes["store"] = wl.store_bytes(layers=1)
            self.reference_bytes["store"] = effective_bytes(
                "store", int(wl.slot_mapping.size), wl.num_kv_heads, wl.head_dim, element)
        if name != "decode_store":
            self.plan = backend.build_gather_plan(self.key_cache, self.tables, self.cu, self.total)
            self.k_out = torch.empty((self.total, wl.num_kv_heads, wl.head_dim), dtype=wl.dtype,
                                     device=self.device)
            self.v_out = torch.empty_like(self.k_out)
            self.ops["gather_varlen_kv"] = lambda: backend.gather_varlen(
                self.key_cache, self.value_cache, self.tables, self.cu, self.total, plan=self.plan,
                out=(self.k_out, self.v_out))
            self.algorithmic_bytes["gather_varlen_kv"] = wl.gather_bytes(layers=1)
            self.reference_bytes["gather_varlen_kv"] = 2 * effective_bytes(
                "gather", self.total, wl.num_kv_heads, wl.head_dim, element)
        if wl.phase == "prefill" and wl.slot_mapping is not None:
            # the same step's store and context gather as one launch
            self.cu_q = torch.from_numpy(wl.cu_seqlens_q()).to(self.device)
            self.sg_plan = backend.build_store_gather_plan(
                self.key_cache, self.tables, self.cu_q, self.cu, self.key.shape[0], self.total)
            self.sg_out = (torch.empty_like(self.k_out), torch.empty_like(self.v_out))
            self.ops["store_gather"] = lambda: backend.store_gather(
                self.key, self.value, self.key_cache, self.value_cache, self.slots, self.tables,
                self.cu_q, self.cu, self.total, plan=self.sg_plan, out=self.sg_out)
            self.algorithmic_bytes["store_gather"] = wl.store_gather_bytes(layers=1)
            self.reference_bytes["store_gather"] = (self.reference_bytes["store"]
                                                    + self.reference_bytes["gather_varlen_kv"])

    def steady_state_us(self, op: str, rotations: int = 16, rounds: int = 4) -> float:
        """Microseconds per launch of ``op`` launched back to back, rotating
        over ``rotations`` disjoint sets: each set has its own inputs (K/V
        rows for the store, outputs for the gather) and its own destination
        or source blocks (every block id shifted by k * num_blocks /
        rotations), so no launch finds its bytes in the MALL and the
        write-backs of earlier launches fall inside later ones.  One event
        pair around rotations x rounds launches; the host enqueues faster
        than the kernels run."""
        import numpy as np

        wl, backend = self.wl, self.backend
        nb, bs = wl.num_blocks, wl.block_size
        shift = max(1, nb // rotations)
        calls = []
        for k in range(rotations):
            if op == "store":
                slots = self.wl.slot_mapping.astype(np.int64)
                moved = np.where(slots >= 0, ((slots // bs + k * shift) % nb) * bs + slots % bs, -1)
                d_slots = torch.from_numpy(moved.astype(np.int32)).to(self.device)
                key, value = self.key.clone(), self.value.clone()
                calls.append(lambda key=key, value=value, d_slots=d_slots: backend.store(
                    key, value, self.key_cache, self.value_cache, d_slots))
            elif op == "store_gather":
                slots = self.wl.slot_mapping.astype(np.int64)
                moved = np.where(slots >= 0, ((slots // bs + k * shift) % nb) * bs + slots % bs, -1)
                d_slots = torch.from_numpy(moved.astype(np.int32)).to(self.device)
                base = self.wl.padded_block_tables().astype(np.int64)
                tables = torch.from_numpy(np.where(base >= 0, (base + k * shift) % nb, -1)
                                          .astype(np.int32)).to(self.device)
                plan = backend.build_store_gather_plan(self.key_cache, tables, self.cu_q, self.cu,
                                                       self.key.shape[0], self.total)
                key, value = self.key.clone(), self.value.clone()
                out = (torch.empty_like(self.k_out), torch.empty_like(self.v_out))
                calls.append(lambda key=key, value=value, d_slots=d_slots, tables=tables, plan=plan,
                             out=out: backend.store_gather(
                                 key, value, self.key_cache, self.value_cache, d_slots, tables,
                                 self.cu_q, self.cu, self.total, plan=plan, out=out))
            elif op == "gather_varlen_kv":
                base = self.wl.padded_block_tables().astype(np.int64)
                tables = torch.from_numpy(np.where(base >= 0, (base + k * shift) % nb, -1)
                                          .astype(np.int32)).to(self.device)
                plan = backend.build_gather_plan(self.key_cache, tables, self.cu, self.total)
                k_out, v_out = torch.empty_like(self.k_out), torch.empty_like(self.v_out)
                calls.append(lambda tables=tables, plan=plan, k_out=k_out, v_out=v_out:
                             backend.gather_varlen(self.key_cache, self.value_cache, tables, self.cu,
                                                   self.total, plan=plan, out=(k_out, v_out)))
            else:
                raise ValueError(f"no steady-state form of {op}")
        for call in calls:
            call()
        torch.cuda.synchronize(self.device)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(rounds):
            for call in calls:
                call()
        end.record()
        torch.cuda.synchronize(self.device)
        return start.elapsed_time(end) * 1e3 / (rounds * rotations)

    def check(self) -> None:
        """Run the step once through the hip backend and once through the
        torch restatement of the reference backend (on copies of the
        caches), and require bit-identical caches and gathered K/V."""
        ref = TorchReferenceBackend()
        words = torch.int16 if self.key_cache.element_size() == 2 else torch.int32
        expect_k, expect_v = self.key_cache.clone(), self.value_cache.clone()
        if "store" in self.ops:
            ref.store(self.key, self.value, expect_k, expect_v, self.slots)
            self.ops["store"]()
            if not (torch.equal(self.key_cache.view(words), expect_k.view(words))
                    and torch.equal(self.value_cache.view(words), expect_v.view(words))):
                raise AssertionError(f"{self.name}: hip store differs from the reference backend")
        if "gather_varlen_kv" in self.ops:
            self.ops["gather_varlen_kv"]()
            starts = self.wl.cu_seqlens_k().tolist()
            for i, n in enumerate(self.context_lens.tolist()):
                table = self.tables[i, : max(1, -(-n // self.wl.block_size))]
                for cache, out in ((expect_k, self.k_out), (expect_v, self.v_out)):
                    got = out[starts[i]:starts[i] + n].view(words)
                    if not torch.equal(got, ref.gather(cache, table, n).view(words)):
                        raise AssertionError(f"{self.name}: hip gather of sequence {i} differs from "
                                             f"the reference backend")
        if "store_gather" in self.ops:
            # the store is idempotent: after it the fused op must leave the
            # same caches and give the reference's gathers of them
            self.ops["store_gather"]()
            if not (torch.equal(self.key_cache.view(words), expect_k.view(words))
                    and torch.equal(self.value_cache.view(words), expect_v.view(words))):
                raise AssertionError(f"{self.name}: hip store+gather leaves other caches")
            starts = self.wl.cu_seqlens_k().tolist()
            for i, n in enumerate(self.context_lens.tolist()):
                table = self.tables[i, : max(1, -(-n // self.wl.block_size))]
                for cache, out in ((expect_k, self.sg_out[0]), (expect_v, self.sg_out[1])):
                    got = out[starts[i]:starts[i] + n].view(words)
                    if not torch.equal(got, ref.gather(cache, table, n).view(words)):
                        raise AssertionError(f"{self.name}: hip store+gather of sequence {i} "
                                             f"differs from the reference backend")
        torch.cuda.synchronize(self.device)


def run_workload(name: str, *, iterations: int = 50, warmup: int = 5, device=None) -> list[dict]:
    """Measure the HIP path on one named workload (nanokv.workloads) and
    return one record per operation: algorithmic bytes, latency summary,
    GB/s at p50 and the fraction of the HBM peak."""
    from nanokv.packing import DevicePacker, SequenceBatch

    device = device or torch.device("cuda", 0)
    prepared = PreparedWorkload(name, device)
    prepared.check()
    wl = prepared.wl
    flush = torch.zeros(FLUSH_BYTES, dtype=torch.uint8, device=device)
    records = []

    def record(op, nbytes, samples, reference_bytes):
        summary = summarize_latencies(samples)
        gbps = nbytes / (summary["p50_us"] * 1e-6) / 1e9 if nbytes else None
        records.append({
            "workload": name, "operation": op, "algorithmic_bytes": nbytes,
            "reference_effective_bytes": reference_bytes, "latency": summary,
            "gbps_at_p50": round(gbps, 2) if gbps else None,
            "hbm_fraction": round(gbps / MI355X_HBM_PEAK_GBPS, 4) if gbps else None,
        })

    def steady(op):
        # A launch moving less than ~8 MB finishes faster than the host can
        # issue the next call (about 10 µs of validation and launch), so a
        # back-to-back rate would time the host; those keep the p50 only.
        if prepared.algorithmic_bytes[op] < (8 << 20):
            return
        us = prepared.steady_state_us(op)
        gbps = prepared.algorithmic_bytes[op] / (us * 1e3)
        records[-1]["steady_state"] = {
            "us_per_launch": round(us, 2), "gbps": round(gbps, 2),
            "hbm_fraction": round(gbps / MI355X_HBM_PEAK_GBPS, 4),
            "method": "16 rotating disjoint input/output sets, launches back to back, one event pair",
        }

    if "store" in prepared.ops:
        record("store", prepared.algorithmic_bytes["store"],
               _time_with_flush(prepared.ops["store"], flush, iterations, warmup),
               prepared.reference_bytes["store"])
        steady("store")
    if "gather_varlen_kv" in prepared.ops:
        offsets, ids = wl.csr()
        packer = DevicePacker(device, wl.block_size)
        batch = SequenceBatch(wl.num_tokens, offsets, ids, wl.num_prompt, wl.num_cached, wl.num_scheduled)
        if wl.phase == "decode":
            record("pack_decode", 0, _time_with_flush(lambda: packer.pack_decode(batch), flush,
                                                      iterations, warmup), 0)
        else:
            record("pack_prefill", 0, _time_with_flush(
                lambda: packer.pack_prefill(batch, force_block_tables=True), flush, iterations, warmup), 0)
        record("gather_varlen_kv", prepared.algorithmic_bytes["gather_varlen_kv"],
               _time_with_flush(prepared.ops["gather_varlen_kv"], flush, iterations, warmup),
               prepared.reference_bytes["gather_varlen_kv"])
        steady("gather_varlen_kv")
        if "store_gather" in prepared.ops:
            record("store_gather", prepared.algorithmic_bytes["store_gather"],
                   _time_with_flush(prepared.ops["store_gather"], flush, iterations, warmup),
                   prepared.reference_bytes["store_gather"])
            steady("store_gather")
        record("build_gather_plan", 0, _time_with_flush(
            lambda: prepared.backend.build_gather_plan(prepared.key_cache, prepared.tables,
                                                       prepared.cu, prepared.total),
            flush, iterations, warmup), 0)
    return records


def replay_workload(name: str, replays: int, device=None) -> None:
    """The profiling replay of one workload: a bit-exact check against the
    reference backend, then ``replays`` rounds of (MALL eviction, each
    operation), with no events, for a profiler to record."""
    device = device or torch.device("cuda", 0)
    prepared = PreparedWorkload(name, device)
    prepared.check()
    flush = torch.zeros(FLUSH_BYTES, dtype=torch.uint8, device=device).view(torch.int64)
    for _ in range(replays):
        for op in prepared.ops.values():
            flush.sum()
            op()
    torch.cuda.synchronize(device)


def replay_store_floor(replays: int, device=None) -> None:
    """The chunked-prefill store beside what bounds it, for a profiler:
    ``replays`` launches each, in this order, of (1) torch's ``copy_`` of a
    32 MiB bf16 tensor, 67,108,864 bytes moved, what the store of 8,192 rows
    of 2 KiB of K and V moves; (2) the store of 8,192 K/V rows into slots
    0..8191 (32 consecutive blocks); (3) the same rows into the
    chunked-prefill workload's slots (blocks scattered over the 2 GiB
    caches).  A 512 MiB read precedes every launch, as in the workload
    replay.  Nothing else launches the store kernel, so a trace splits its
    dispatches between (2) and (3) by order; both stores' results are
    checked bit-exactly by the GPU parity tests, not here."""
    from nanokv import workloads
    from nanokv.paged_kv import create_paged_kv_backend

    device = device or torch.device("cuda", 0)
    backend = create_paged_kv_backend("hip")
    wl = workloads.build("chunked_prefill")
    shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
    g = torch.Generator(device=device).manual_seed(23)
    key_cache = torch.randn(shape, generator=g, device=device).to(wl.dtype)
    value_cache = torch.randn(shape, generator=g, device=device).to(wl.dtype)
    rows = (wl.slot_mapping.size, wl.num_kv_heads, wl.head_dim)
    key = torch.randn(rows, generator=g, device=device).to(wl.dtype)
    value = torch.randn(rows, generator=g, device=device).to(wl.dtype)
    contiguous = torch.arange(rows[0], dtype=torch.int32, device=device)
    scattered = torch.from_numpy(wl.slot_mapping).to(device)
    src = torch.randn(key.numel() * 2, generator=g, device=device).to(wl.dtype)
    dst = torch.empty_like(src)
    assert 2 * src.numel() * src.element_size() == 67_108_864
    ops = (lambda: dst.copy_(src),
           lambda: backend.store(key, value, key_cache, value_cache, contiguous),
           lambda: backend.store(key, value, key_cache, value_cache, scattered))
    flush = torch.zeros(FLUSH_BYTES, dtype=torch.uint8, device=device).view(torch.int64)
    torch.cuda.synchronize(device)
    for op in ops:
        for _ in range(replays):
            flush.sum()
            op()
    torch.cuda.synchronize(device)


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
            json.dump({"schema_version": "nanokv.paged_kv_workloads.v1",
                       "identity": environment_identity(torch.device("cuda", 0)),
                       "records": records}, handle, indent=1)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
