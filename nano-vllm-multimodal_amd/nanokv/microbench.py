"""Store / gather micro-benchmark of the paged-KV backends: a case matrix,
a bit-exactness gate before any timing, per-call event timing, and JSON +
Markdown reports written atomically.

The command line, the case selector, the report's schema id and its field
names are the reference's (bench_paged_kv.py:58-148,
nanovllm/benchmark/paged_kv.py:28-101,142-214,364-394), so its scripts and
report readers work unchanged.  The backends measured here are ``hip``
(this library) and ``pytorch`` (the reference's pytorch backend's torch
ops, :class:`nanokv.benchmark.TorchReferenceBackend`); the reference's
``triton`` and ``cuda`` backends are not built on this platform and are
rejected by name.

    python -m nanokv.microbench [--backends hip,pytorch] [--operations store,gather]
        [--dtypes float16,bfloat16] [--tokens 1,8,257] [--kv-shapes 1x64,2x128,8x128]
        [--num-blocks 64] [--block-size 16]
        [--mapping contiguous|random|random_with_skips] [--seed 17]
        [--warmup 100] [--iterations 1000] [--device cuda:0]
        [--case-selector SELECTOR [--profile-replay N]] [--output-dir DIR]

A case runs on its own cache of ``num_blocks`` x ``block_size`` slots
filled from N(0, 1).  K and V are N(0, 1) rows from a generator seeded with
the case seed; the slot mapping is 0..T-1 (contiguous) or the first T of a
random permutation of the cache's slots (random), every 11th then set to -1
(random_with_skips); the gather reads T rows through a random permutation
of the blocks.  Before it is timed, every case's result is compared word
for word with the reference's torch ops on the same inputs.
"""
from __future__ import annotations

import argparse
import json
import os
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Callable, Iterable, Sequence

import torch

from nanokv.benchmark import (
    TorchReferenceBackend,
    effective_bytes,
    environment_identity,
    summarize_latencies,
)

SCHEMA = "nanoinfer.paged_kv_benchmark.v1"
BACKENDS = ("hip", "pytorch")
NOT_BUILT = ("triton", "cuda")  # the reference's other backends
OPERATIONS = ("store", "gather")
MAPPINGS = ("contiguous", "random", "random_with_skips")
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
DTYPE_NAMES = {dtype: name for name, dtype in DTYPES.items()}
REPORT_STEM = "paged-kv-microbenchmark"
# selector keys in their order, with the case field each one fills
SELECTOR_FIELDS = (("backend", "backend"), ("operation", "operation"), ("dtype", "dtype"),
                   ("tokens", "num_tokens"), ("blocks", "num_blocks"), ("block", "block_size"),
                   ("heads", "num_kv_heads"), ("dim", "head_dim"), ("mapping", "mapping"),
                   ("seed", "seed"))


@dataclass(frozen=True)
class Case:
    """One benchmark case; invalid combinations raise ValueError."""

    backend: str
    operation: str
    dtype: torch.dtype
    num_tokens: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    mapping: str = "contiguous"
    seed: int = 17

    def __post_init__(self) -> None:
        if self.backend in NOT_BUILT:
            raise ValueError(f"the {self.backend} backend is not built on this platform; "
                             f"backends here: {', '.join(BACKENDS)}")
        if self.backend not in BACKENDS:
            raise ValueError(f"unsupported Paged KV backend: {self.backend}")
        if self.operation not in OPERATIONS:
            raise ValueError(f"unsupported Paged KV operation: {self.operation}")
        if self.dtype not in DTYPE_NAMES:
            raise ValueError(f"unsupported Paged KV dtype: {self.dtype}")
        sizes = (self.num_tokens, self.num_blocks, self.block_size, self.num_kv_heads,
                 self.head_dim)
        if min(sizes) <= 0:
            raise ValueError("Paged KV benchmark dimensions must be positive")
        if self.num_tokens > self.num_blocks * self.block_size:
            raise ValueError("num_tokens exceeds Paged KV cache capacity")
        if self.mapping not in MAPPINGS:
            raise ValueError(f"unsupported slot mapping: {self.mapping}")

    @property
    def selector(self) -> str:
        """``key=value`` pairs joined by ``;``, every identity field."""
        values = {"dtype": DTYPE_NAMES[self.dtype]}
        return ";".join(f"{key}={values.get(key, getattr(self, attr))}"
                        for key, attr in SELECTOR_FIELDS)

    @classmethod
    def from_selector(cls, selector: str) -> "Case":
        try:
            pairs = [part.split("=", 1) for part in selector.split(";")]
            given = {key: value for key, value in pairs}
            if len(given) != len(pairs) or set(given) != {key for key, _ in SELECTOR_FIELDS}:
                raise ValueError
            kwargs: dict[str, Any] = {}
            for key, attr in SELECTOR_FIELDS:
                raw = given[key]
                if key == "dtype":
                    kwargs[attr] = DTYPES[raw]
                elif key in ("backend", "operation", "mapping"):
                    kwargs[attr] = raw
                else:
                    kwargs[attr] = int(raw)
        except (KeyError, TypeError, ValueError) as exc:
            raise ValueError(f"invalid Paged KV case selector: {selector}") from exc
        return cls(**kwargs)

    def to_dict(self) -> dict[str, Any]:
        record = {attr: getattr(self, attr) for _, attr in SELECTOR_FIELDS}
        record["dtype"] = DTYPE_NAMES[self.dtype]
        record["selector"] = self.selector
        return record


def expand_matrix(*, backends: Sequence[str], operations: Sequence[str],
                  dtypes: Sequence[torch.dtype], token_counts: Sequence[int],
                  kv_shapes: Sequence[tuple[int, int]], block_size: int, num_blocks: int,
                  mapping: str = "random_with_skips", seed: int = 17) -> tuple[Case, ...]:
    """Every combination, backend outermost and token count innermost (the
    reference's order, so case i means the same case in both reports)."""
    return tuple(Case(backend, operation, dtype, tokens, num_blocks, block_size, heads, dim,
                      mapping, seed)
                 for backend in backends for operation in operations for dtype in dtypes
                 for heads, dim in kv_shapes for tokens in token_counts)


def case_effective_bytes(case: Case) -> int:
    """The reference's byte count: the K+V payload x 4 for a store (read and
    write), x 2 for a gather of one cache, -1 slots included."""
    element = torch.empty((), dtype=case.dtype).element_size()
    return effective_bytes(case.operation, case.num_tokens, case.num_kv_heads, case.head_dim,
                           element)


@dataclass
class Prepared:
    """A case's tensors on the device and its one call."""

    case: Case
    backend: Any
    key: torch.Tensor
    value: torch.Tensor
    key_cache: torch.Tensor
    value_cache: torch.Tensor
    slot_mapping: torch.Tensor
    block_table: torch.Tensor
    owner: Any = None
    reference: TorchReferenceBackend = field(default_factory=TorchReferenceBackend)

    def invoke(self) -> torch.Tensor | None:
        if self.case.operation == "store":
            self.backend.store(self.key, self.value, self.key_cache, self.value_cache,
                               self.slot_mapping)
            return None
        return self.backend.gather(self.key_cache, self.block_table, self.case.num_tokens)

    def check(self) -> None:
        """One call against the reference's torch ops on the same inputs,
        compared as integer words (bit-exact; NaN-safe)."""
        word = torch.int32 if self.case.dtype == torch.float32 else torch.int16
        if self.case.operation == "store":
            expect_k, expect_v = self.key_cache.clone(), self.value_cache.clone()
            self.reference.store(self.key, self.value, expect_k, expect_v, self.slot_mapping)
            self.invoke()
            torch.cuda.synchronize(self.key.device)
            if not torch.equal(self.key_cache.view(word), expect_k.view(word)):
                raise AssertionError(f"{self.case.selector}: key cache differs from the reference")
            if not torch.equal(self.value_cache.view(word), expect_v.view(word)):
                raise AssertionError(f"{self.case.selector}: value cache differs from the reference")
            return
        expect = self.reference.gather(self.key_cache, self.block_table, self.case.num_tokens)
        got = self.invoke()
        torch.cuda.synchronize(self.key_cache.device)
        if got is None or not torch.equal(got.view(word), expect.view(word)):
            raise AssertionError(f"{self.case.selector}: gather differs from the reference")


def prepare(case: Case, device: torch.device | str = "cuda") -> Prepared:
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("the Paged KV micro-benchmark runs on a GPU device")
    from nanokv.paged_kv import create_paged_kv_backend

    shape = (2, case.num_blocks, case.block_size, case.num_kv_heads, case.head_dim)
    owner = None
    if case.backend == "hip":
        backend = create_paged_kv_backend("hip")
        allocation = backend.allocate(shape, dtype=case.dtype, device=device)
        cache, owner = allocation.tensor, allocation.owner
    else:
        backend = TorchReferenceBackend()
        cache = torch.empty(shape, dtype=case.dtype, device=device)
    cache.normal_()
    g = torch.Generator(device=device)
    g.manual_seed(case.seed)
    rows = (case.num_tokens, case.num_kv_heads, case.head_dim)
    key = torch.randn(rows, dtype=case.dtype, device=device, generator=g)
    value = torch.randn(rows, dtype=case.dtype, device=device, generator=g)
    if case.mapping == "contiguous":
        slots = torch.arange(case.num_tokens, dtype=torch.int32, device=device)
    else:
        capacity = case.num_blocks * case.block_size
        slots = torch.randperm(capacity, dtype=torch.int32, device=device,
                               generator=g)[:case.num_tokens].contiguous()
        if case.mapping == "random_with_skips":
            slots[::11] = -1
    table = torch.randperm(case.num_blocks, dtype=torch.int32, device=device, generator=g)
    torch.cuda.synchronize(device)
    return Prepared(case, backend, key, value, cache[0], cache[1], slots, table, owner)


def time_calls(invoke: Callable[[], Any], iterations: int) -> list[float]:
    """Microseconds of each of ``iterations`` calls, one event pair around
    each on the current stream (the reference's per-iteration method)."""
    if iterations <= 0:
        raise ValueError("iterations must be positive")
    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(iterations)]
    for start, end in pairs:
        start.record()
        invoke()
        end.record()
    pairs[-1][1].synchronize()
    return [start.elapsed_time(end) * 1000.0 for start, end in pairs]


def gated(check: Callable[[], None], warm: Callable[[], None],
          measure: Callable[[], list[float]]) -> list[float]:
    """Correctness first, then warm-up, then the timed calls: a case that
    fails its check is never timed."""
    check()
    warm()
    return measure()


def run_case(case: Case, *, warmup: int = 100, iterations: int = 1000,
             device: torch.device | str = "cuda") -> dict[str, Any]:
    if warmup < 0:
        raise ValueError("warmup iterations must be non-negative")
    prepared = prepare(case, device)

    def warm() -> None:
        for _ in range(warmup):
            prepared.invoke()
        torch.cuda.synchronize(device)

    samples = gated(prepared.check, warm, lambda: time_calls(prepared.invoke, iterations))
    latency = summarize_latencies(samples)
    nbytes = case_effective_bytes(case)
    p50 = latency["p50_us"]
    return {
        "case": case.to_dict(),
        "correctness": "pass",
        "warmup_iterations": warmup,
        "iterations": iterations,
        "effective_bytes": nbytes,
        "effective_gbps_at_p50": nbytes / (p50 * 1000.0) if p50 > 0 else 0.0,
        "latency": latency,
        "samples_us": samples,
    }


def build_report(results: Iterable[dict[str, Any]], device: torch.device | str = "cuda") -> dict:
    return {"schema_version": SCHEMA, "identity": environment_identity(torch.device(device)),
            "results": list(results)}


def render_markdown(report: dict[str, Any]) -> str:
    lines = [f"# Paged KV micro-benchmark ({report['schema_version']})", "",
             f"GPU: {report['identity'].get('gpu_name', 'unknown')} "
             f"({report['identity'].get('gpu_arch', '')}), torch {report['identity'].get('torch')}", "",
             "| Backend | Operation | Dtype | Tokens | KV shape | Mapping | p50 (us) | p95 (us) "
             "| p99 (us) | GB/s at p50 | Correctness |",
             "|---|---|---|---:|---|---|---:|---:|---:|---:|---|"]
    for r in report["results"]:
        c, lat = r["case"], r["latency"]
        lines.append(f"| {c['backend']} | {c['operation']} | {c['dtype']} | {c['num_tokens']} | "
                     f"{c['num_kv_heads']}x{c['head_dim']} | {c['mapping']} | {lat['p50_us']:.2f} | "
                     f"{lat['p95_us']:.2f} | {lat['p99_us']:.2f} | {r['effective_gbps_at_p50']:.2f} | "
                     f"{r['correctness']} |")
    return "\n".join(lines) + "\n"


def _atomic_write(path: Path, text: str) -> None:
    """Write ``text`` to a temporary file beside ``path``, flush it to disk,
    then rename it over ``path``: a reader sees the old file or the whole
    new one, never a partial write."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    temporary = path.with_name(f".{path.name}.{os.getpid()}.tmp")
    try:
        with open(temporary, "w", encoding="utf-8") as handle:
            handle.write(text)
            handle.flush()
            os.fsync(handle.fileno())
        os.replace(temporary, path)
    finally:
        if temporary.exists():
            temporary.unlink()


def write_json_atomic(path: Path, payload: Any) -> None:
    _atomic_write(path, json.dumps(payload, indent=2, sort_keys=True) + "\n")


def write_text_atomic(path: Path, text: str) -> None:
    _atomic_write(path, text)


# ---------------------------------------------------------------- command line

def _csv(value: str) -> tuple[str, ...]:
    items = tuple(part.strip() for part in value.split(",") if part.strip())
    if not items:
        raise argparse.ArgumentTypeError("expected a non-empty comma-separated list")
    return items


def _positive_ints(value: str) -> tuple[int, ...]:
    try:
        items = tuple(int(part) for part in _csv(value))
    except ValueError as exc:
        raise argparse.ArgumentTypeError("expected comma-separated integers") from exc
    if min(items) <= 0:
        raise argparse.ArgumentTypeError("integer matrix values must be positive")
    return items


def _kv_shapes(value: str) -> tuple[tuple[int, int], ...]:
    shapes = []
    for part in _csv(value):
        heads, sep, dim = part.lower().partition("x")
        try:
            shape = (int(heads), int(dim))
        except ValueError as exc:
            raise argparse.ArgumentTypeError("KV shapes must use HEADSxDIM") from exc
        if not sep or min(shape) <= 0:
            raise argparse.ArgumentTypeError("KV shapes must use positive HEADSxDIM")
        shapes.append(shape)
    return tuple(shapes)


def build_parser() -> argparse.ArgumentParser:
    p = argparse.ArgumentParser(prog="python -m nanokv.microbench", description=__doc__,
                                formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--backends", type=_csv, default=BACKENDS)
    p.add_argument("--operations", type=_csv, default=OPERATIONS)
    p.add_argument("--dtypes", type=_csv, default=("float16", "bfloat16"))
    p.add_argument("--tokens", type=_positive_ints, default=(1, 8, 257))
    p.add_argument("--kv-shapes", type=_kv_shapes, default=((1, 64), (2, 128), (8, 128)))
    p.add_argument("--num-blocks", type=int, default=64)
    p.add_argument("--block-size", type=int, default=16)
    p.add_argument("--mapping", choices=MAPPINGS, default="random_with_skips")
    p.add_argument("--seed", type=int, default=17)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--iterations", type=int, default=1000)
    p.add_argument("--device", default="cuda:0")
    p.add_argument("--case-selector", help="run only this case (a selector from a report)")
    p.add_argument("--profile-replay", type=int, default=0, metavar="N",
                   help="with --case-selector: check the case once, then call it N times with "
                        "no events, for a profiler")
    p.add_argument("--output-dir", type=Path, default=Path("benchmark-results/paged-kv"))
    return p


def resolve_cases(args: argparse.Namespace) -> tuple[Case, ...]:
    if args.case_selector:
        return (Case.from_selector(args.case_selector),)
    unknown = [name for name in args.dtypes if name not in DTYPES]
    if unknown:
        raise ValueError(f"unsupported dtypes: {', '.join(unknown)}")
    return expand_matrix(backends=args.backends, operations=args.operations,
                         dtypes=tuple(DTYPES[n] for n in args.dtypes), token_counts=args.tokens,
                         kv_shapes=args.kv_shapes, block_size=args.block_size,
                         num_blocks=args.num_blocks, mapping=args.mapping, seed=args.seed)


def main(argv: Sequence[str] | None = None) -> int:
    args = build_parser().parse_args(argv)
    if args.profile_replay < 0:
        raise ValueError("--profile-replay must be non-negative")
    if args.profile_replay and not args.case_selector:
        raise ValueError("--profile-replay needs exactly one --case-selector")
    cases = resolve_cases(args)
    if not torch.cuda.is_available():
        raise RuntimeError("the Paged KV micro-benchmark needs a visible ROCm GPU")
    if args.profile_replay:
        prepared = prepare(cases[0], args.device)
        prepared.check()
        for _ in range(args.profile_replay):
            prepared.invoke()
        torch.cuda.synchronize(args.device)
        print(f"profile replay complete: {cases[0].selector}", flush=True)
        return 0
    results = []
    for index, case in enumerate(cases, 1):
        print(f"[{index}/{len(cases)}] {case.selector}", flush=True)
        results.append(run_case(case, warmup=args.warmup, iterations=args.iterations,
                                device=args.device))
    report = build_report(results, args.device)
    json_path = args.output_dir / f"{REPORT_STEM}.json"
    markdown_path = args.output_dir / f"{REPORT_STEM}.md"
    write_json_atomic(json_path, report)
    write_text_atomic(markdown_path, render_markdown(report))
    print(f"wrote {json_path}\nwrote {markdown_path}", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
