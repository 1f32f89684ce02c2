#!/usr/bin/env python3
"""Paged-KV decode-step benchmark on one MI355X.

One step = the device packs the step's metadata (slot_mapping, context
lengths, -1 padded block tables, cu_seqlens_k) from the scheduler's
per-sequence CSR state, builds the gather plan, then for each of the 28
layers stores the 256 new K/V rows into the paged cache and gathers every
sequence's K and V context into contiguous varlen buffers (one launch per
layer).  Workload: Qwen3-VL-2B language-model KV shape (8 kv heads x 128,
bf16), 256 live sequences with contexts log-uniform in [256, 16384] after
16 evictions and 16 admissions, cache [2, 28, blocks, 256, 8, 128].

Prints one JSON line:  value = store+gather algorithmic GB/s of the step
(sum of the bytes the store and gather must move / step time), plus
decode tokens/s, the HBM roofline of the dominant kernel (the varlen
gather, timed live with events on its stream, and checked against a
rocprofv3 kernel trace of the same step taken on the same host before the
timed run, "rocprof_same_host") and a CPU baseline: the
reference pytorch backend's torch ops (index_copy_ store, index_select
gather) on host tensors with every host thread, over the same step and the
single-layer configurations, with the oracle's OpenMP C restatement timed
beside it as a second figure.  The same leg first checks the GPU outputs
of --check-layers against the oracle (store+gather bit-exact, attention
within tolerance).  A second
timed step replaces the gather by its consumer, paged-attention decode read
straight from the cache (16 query heads), reported under "attention", and
"block_pool" times the same steps' block bookkeeping replayed on the device
block pool (with the host restatement's time in the CPU leg).
"copy_reference" times a plain device copy of the gather's payload and the
gather over contiguous block tables; "other_workloads" times the
single-layer store / gather configurations (decode store, chunked-prefill
store, prefix-cache gather, narrow rows) kernel by kernel; "gpu_reference"
runs the reference pytorch backend's torch ops on the same GPU, on the
decode step and on the reference's own store/gather microbenchmark matrix;
"prefill_attention" (with --prefill-attention) times the causal paged
prefill kernel on the chunked-prefill step against the reference's SDPA
prefill path;
"grouped_decode_attention" times one decode-attention layer over the same
contexts for the grouped-query layouts of Qwen2.5-VL-3B / -7B and
Qwen3-VL-8B (the MFMA decode kernel).
"""
from __future__ import annotations

import argparse
import json
import math
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
for _p in (REPO_ROOT, REPO_ROOT / "nano-vllm-multimodal_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "paged KV store+gather GB/s (fraction of HBM peak); decode-step tokens/s, 1 GPU"
# Cases of the profiling replay (--case): the four single-layer
# configurations, the full decode step (store + gather) and the decode step
# with paged-attention decode in place of the gather.
PROFILE_CASES = ("decode_store", "chunked_prefill", "prefix_gather", "narrow_rows", "decode_step",
                 "decode_attention", "grouped_decode_2x8", "grouped_decode_4x7", "grouped_decode_8x4",
                 "prefill_attention", "block_pool", "store_floor")


PROFILE_FILE = REPO_ROOT / "profiles" / "decode_step_rocprof.json"
ATTENTION_PROFILE_FILE = REPO_ROOT / "profiles" / "decode_attention_rocprof.json"


def profiled_median(path: Path, kernel_prefix: str, algorithmic_bytes: int):
    """Median per-dispatch duration (µs) of a kernel in a committed
    rocprofv3 summary (written by ``python -m nanokv.profiling report``),
    or None unless it was profiled on this workload (same algorithmic
    bytes per launch)."""
    if not path.is_file():
        return None
    try:
        kernels = json.loads(path.read_text()).get("kernels", {})
    except (OSError, ValueError):
        return None
    for name, record in kernels.items():
        if name.startswith(kernel_prefix) and record.get("algorithmic_bytes") == algorithmic_bytes:
            return round(record["median_us"], 2)
    return None


def measured_traffic(path: Path, kernel_prefix: str, algorithmic_bytes: int):
    """HBM bytes per launch of a kernel (FETCH_SIZE + WRITE_SIZE, each scaled
    by its reading for a copy of known size) from a committed rocprofv3
    summary, or None unless the summary was taken on this workload (same
    algorithmic bytes per launch)."""
    if not path.is_file():
        return None
    try:
        kernels = json.loads(path.read_text()).get("kernels", {})
    except (OSError, ValueError):
        return None
    for name, record in kernels.items():
        if (name.startswith(kernel_prefix) and record.get("algorithmic_bytes") == algorithmic_bytes
                and "traffic_bytes" in record):
            return record["traffic_bytes"]
    return None


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--layers", type=int, default=28)
    p.add_argument("--check-layers", default="0", help="comma list of layers checked vs the oracle; '' = none")
    p.add_argument("--cpu-baseline-layers", type=int, default=28,
                   help="decode-step layers in the CPU baseline sample of the reference's torch "
                        "ops (0 disables the CPU leg)")
    p.add_argument("--cpu-baseline-repeats", type=int, default=3,
                   help="runs of the 28-layer step in the OpenMP port's figure")
    p.add_argument("--cpu-baseline-runs", type=int, default=5,
                   help="runs of the sampled decode step through the reference's torch ops; "
                        "the median run is reported (about 2 s each on 16 cores)")
    p.add_argument("--workload-iterations", type=int, default=30,
                   help="timed launches per operation of the single-layer configurations; 0 = skip")
    p.add_argument("--no-gpu-reference", dest="gpu_reference", action="store_false",
                   help="skip the torch restatement of the reference pytorch backend on the GPU")
    p.add_argument("--profile", action="store_true",
                   help="run warmup + timed steps only (no check, no CPU baseline), for rocprofv3")
    p.add_argument("--prefill-only", action="store_true",
                   help="only time the paged prefill attention on the chunked-prefill step "
                        "(and its SDPA-path baseline), print that record, then exit")
    p.add_argument("--prefill-attention", action="store_true",
                   help="also time the paged prefill attention in the default run (off by default: "
                        "prefill attention is outside the store/gather path)"),
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="only run a plain device copy of this many MiB 3 times (the known-size "
                        "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE), then exit")
    p.add_argument("--case", choices=PROFILE_CASES,
                   help="with --profile-replay: the one case to replay for a profiler")
    p.add_argument("--profile-replay", type=int, default=0, metavar="N",
                   help="check --case once against the reference backend, replay it N times "
                        "with no events (a MALL eviction before every launch of the single-layer "
                        "cases), print one line, exit")
    p.add_argument("--cpu-baseline-workloads", default="decode_store,chunked_prefill,prefix_gather,narrow_rows",
                   help="single-layer configurations the CPU baseline also times ('' = none)")
    p.add_argument("--settle-s", type=float, default=8.0,
                   help="seconds the GPU idles after the decode-step cache is filled, before "
                        "anything is timed (0 = none)")
    p.add_argument("--no-rocprof-check", dest="rocprof_check", action="store_false",
                   help="skip the same-host rocprofv3 kernel trace of the decode step that the "
                        "roofline is checked against")
    args = p.parse_args(argv)
    if bool(args.case) != bool(args.profile_replay):
        p.error("--case and --profile-replay go together")
    if args.profile_replay < 0:
        p.error("--profile-replay must be positive")
    return args


def same_host_roofline(trace: dict | None, launch_bytes: int, launch_us: float) -> dict | None:
    """The gather's figures from the kernel trace taken on this host
    (``nanokv.profiling.trace_kernel_here``): mean and median duration over
    the replay's 280 launches, the fraction of peak at the mean, and the
    ratio of the event-timed back-to-back duration to the trace's mean."""
    if trace is None:
        return None
    if "error" in trace:
        return {"error": trace["error"]}
    from nanokv.benchmark import MI355X_HBM_PEAK_GBPS

    return {
        "kernel": trace["kernel"],
        "dispatches": trace["dispatches"],
        "mean_us": round(trace["mean_us"], 2),
        "median_us": round(trace["median_us"], 2),
        "frac_at_mean": round(launch_bytes / (trace["mean_us"] * 1e3) / MI355X_HBM_PEAK_GBPS, 4),
        "events_over_trace_mean": round(launch_us / trace["mean_us"], 4),
        "command": trace["command"],
    }


def reference_backend():
    """The torch restatement of the reference pytorch backend
    (nanokv.benchmark.TorchReferenceBackend)."""
    from nanokv.benchmark import TorchReferenceBackend

    return TorchReferenceBackend()


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the paged-KV store/gather path is rank-local: under tensor parallelism each rank "
              "runs it on its own kv heads with the same slot_mapping and block tables)",
              file=sys.stderr)
        return 2

    # The decode step's kernel trace on this host, for the roofline's
    # cross-check: a rocprofv3 child process that replays the step, run
    # before this process touches the GPU (so the child has the whole HBM).
    same_host_trace = None
    if (args.rocprof_check and not args.case and not args.profile and not args.prefill_only
            and not args.copy_calibration_mib and args.layers == 28):
        from nanokv.profiling import trace_kernel_here

        log("[bench] rocprofv3 kernel trace of the decode step on this host")
        same_host_trace = trace_kernel_here("decode_step", "gather_planned_kernel", replay=10,
                                            settle_s=args.settle_s, timeout_s=240, echo=True)
        log(f"[bench] same-host trace: {same_host_trace.get('median_us', same_host_trace.get('error'))}")

    import numpy as np
    import torch

    from nanokv import workloads
    from nanokv.benchmark import (MI355X_HBM_PEAK_GBPS, LaunchTimer, effective_bytes, environment_identity,
                                  summarize_latencies)
    from nanokv.packing import DevicePacker, SequenceBatch
    from nanokv.paged_kv import create_paged_kv_backend

    if torch.version.hip is None or not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a ROCm GPU")
    device = torch.device("cuda", 0)
    if args.copy_calibration_mib:
        n = args.copy_calibration_mib << 20
        src = torch.ones(n // 2, dtype=torch.int16, device=device)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": 3}), flush=True)
        return 0
    backend = create_paged_kv_backend("hip")
    if args.case in ("decode_store", "chunked_prefill", "prefix_gather", "narrow_rows"):
        from nanokv.benchmark import replay_workload

        replay_workload(args.case, args.profile_replay, device)
        print(f"profile replay complete: {args.case} x {args.profile_replay}", flush=True)
        return 0
    if args.case == "store_floor":
        from nanokv.benchmark import replay_store_floor

        replay_store_floor(args.profile_replay, device)
        print(f"profile replay complete: store_floor x {args.profile_replay}", flush=True)
        return 0
    if args.case in GROUPED_CASES:
        from nanokv import workloads

        hkv, group = GROUPED_CASES[args.case]
        case = grouped_decode_setup(device, backend, workloads.build("decode_step", num_layers=1),
                                    hkv, group, torch.Generator(device=device).manual_seed(29))
        check_decode_attention(backend, case, sample=6)
        for _ in range(args.profile_replay):
            case["call"]()
        torch.cuda.synchronize(device)
        print(f"profile replay complete: {args.case} x {args.profile_replay}", flush=True)
        return 0
    if args.case == "block_pool":
        from nanokv import workloads
        from nanokv.packing import DevicePacker

        replay_block_pool(workloads.build("decode_step", num_layers=1), device,
                          DevicePacker(device, workloads.BLOCK_SIZE), args.profile_replay)
        print(f"profile replay complete: block_pool x {args.profile_replay}", flush=True)
        return 0
    if args.case == "prefill_attention":
        case = prefill_setup(device, backend)
        check_prefill_attention(backend, case)
        for _ in range(args.profile_replay):
            case["call"]()
        torch.cuda.synchronize(device)
        print(f"profile replay complete: prefill_attention x {args.profile_replay}", flush=True)
        return 0
    if args.prefill_only:
        print(json.dumps(measure_prefill_attention(device, backend, args.steps)), flush=True)
        return 0

    wl = workloads.build("decode_step", num_layers=args.layers)
    L, B = wl.num_layers, wl.num_seqs
    log(f"[bench] decode_step layers={L} seqs={B} blocks={wl.num_blocks} "
        f"context_tokens={int(wl.num_tokens.sum())}")
    cache = torch.empty((2, L, wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim),
                        dtype=wl.dtype, device=device)
    g = torch.Generator(device=device).manual_seed(workloads.seed_for("decode_step"))
    for kv in range(2):
        for layer in range(L):
            cache[kv, layer].normal_(generator=g)
    if args.settle_s > 0:
        # The GPU idles before anything is timed: for a few seconds after a
        # process frees a large allocation (the GPU tests, the trace child
        # above), other GPU activity takes about 3% of HBM bandwidth
        # (gathers 1,192-1,203 against 1,154-1,170 us for ~3.5 s after a
        # process freed 120 GB; no slow phase after a 10 s wait).
        torch.cuda.synchronize(device)
        time.sleep(args.settle_s)
    new_k = wl.key.to(device)
    new_v = wl.value.to(device)
    offsets, ids = wl.csr()
    batch = SequenceBatch(wl.num_tokens, offsets, ids)
    packer = DevicePacker(device, wl.block_size)
    total = int(wl.num_tokens.astype(np.int64).sum())
    k_out = torch.empty((total, wl.num_kv_heads, wl.head_dim), dtype=wl.dtype, device=device)
    v_out = torch.empty_like(k_out)
    stream = torch.cuda.current_stream(device)

    def step(timer: LaunchTimer | None = None, store_timer: LaunchTimer | None = None):
        ctx = packer.pack_decode(batch)
        plan = backend.build_gather_plan(cache[0, 0], ctx.block_tables, ctx.cu_seqlens_k, total)
        for layer in range(L):
            kc, vc = cache[0, layer], cache[1, layer]
            s0 = store_timer.start() if store_timer else None
            backend.store(new_k[layer], new_v[layer], kc, vc, ctx.slot_mapping)
            if store_timer:
                store_timer.stop(s0)
            t0 = timer.start() if timer else None
            backend.gather_varlen(kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total,
                                  plan=plan, out=(k_out, v_out))
            if timer:
                timer.stop(t0)
        return ctx

    # Decode attention straight from the paged cache (the consumer of the
    # gathered K/V): Qwen3-VL-2B's language model has 16 query heads over the
    # 8 kv heads.  Its plan depends on the context lengths only.
    num_q_heads = 16
    softmax_scale = 1.0 / math.sqrt(wl.head_dim)
    q = torch.randn((B, num_q_heads, wl.head_dim), generator=g, device=device).to(wl.dtype)
    attn_out = torch.empty_like(q)

    def attention_step(timer: LaunchTimer | None = None):
        ctx = packer.pack_decode(batch)
        aplan = backend.build_attention_plan(cache[0, 0], ctx.cu_seqlens_k, total)
        for layer in range(L):
            kc, vc = cache[0, layer], cache[1, layer]
            backend.store(new_k[layer], new_v[layer], kc, vc, ctx.slot_mapping)
            t0 = timer.start() if timer else None
            backend.paged_attention_decode(q, kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total,
                                           softmax_scale, plan=aplan, out=attn_out)
            if timer:
                timer.stop(t0)
        return ctx

    host_cu = wl.cu_seqlens_k().tolist()

    def check_layer(layer: int) -> None:
        """Layer ``layer`` of the step (store, then varlen gather) against
        the torch restatement of the reference backend on copies of the
        layer's caches, bit-exact."""
        ref = reference_backend()
        ctx = packer.pack_decode(batch)
        kc, vc = cache[0, layer], cache[1, layer]
        expect_k, expect_v = kc.clone(), vc.clone()
        ref.store(new_k[layer], new_v[layer], expect_k, expect_v, ctx.slot_mapping)
        plan = backend.build_gather_plan(kc, ctx.block_tables, ctx.cu_seqlens_k, total)
        backend.store(new_k[layer], new_v[layer], kc, vc, ctx.slot_mapping)
        backend.gather_varlen(kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total, plan=plan,
                              out=(k_out, v_out))
        words = torch.int16
        if not (torch.equal(kc.view(words), expect_k.view(words))
                and torch.equal(vc.view(words), expect_v.view(words))):
            raise AssertionError(f"decode step layer {layer}: store differs from the reference backend")
        for i, n in enumerate(wl.num_tokens.tolist()):
            for expect, out in ((expect_k, k_out), (expect_v, v_out)):
                got = out[host_cu[i]:host_cu[i] + n].view(words)
                if not torch.equal(got, ref.gather(expect, ctx.block_tables[i], n).view(words)):
                    raise AssertionError(f"decode step layer {layer}: gather of sequence {i} differs")
        del expect_k, expect_v

    def check_attention(layer: int, sample: int = 8) -> None:
        """Paged-attention decode of ``sample`` sequences of layer
        ``layer`` against a float32 softmax(q K^T) V on the host over the
        same K/V rows (gathered bit-exactly above)."""
        ctx = packer.pack_decode(batch)
        kc, vc = cache[0, layer], cache[1, layer]
        backend.gather_varlen(kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total, out=(k_out, v_out))
        backend.paged_attention_decode(q, kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total,
                                       softmax_scale, out=attn_out)
        torch.cuda.synchronize(device)
        group = num_q_heads // wl.num_kv_heads
        for i in np.linspace(0, B - 1, sample).astype(int).tolist():
            lo, n = host_cu[i], int(wl.num_tokens[i])
            # [heads, rows, dim] per query head (kv head h // group), float32 on the host
            keys = k_out[lo:lo + n].float().cpu().repeat_interleave(group, dim=1).transpose(0, 1)
            values = v_out[lo:lo + n].float().cpu().repeat_interleave(group, dim=1).transpose(0, 1)
            query = q[i].float().cpu().unsqueeze(-1)
            weights = torch.softmax(torch.matmul(keys, query).squeeze(-1) * softmax_scale, dim=-1)
            expect = torch.matmul(weights.unsqueeze(1), values).squeeze(1)
            expect_abs = torch.matmul(weights.unsqueeze(1), values.abs()).squeeze(1)
            err = (attn_out[i].float().cpu() - expect).abs()
            if bool((err > attention_tolerance(expect, expect_abs)).any()):
                raise AssertionError(f"decode attention, sequence {i}: max error {float(err.max()):.3e}")

    if args.case == "decode_step":
        check_layer(0)
        for _ in range(args.profile_replay):
            step()
        torch.cuda.synchronize(device)
        print(f"profile replay complete: decode_step x {args.profile_replay}", flush=True)
        return 0
    if args.case == "decode_attention":
        check_attention(0)
        for _ in range(args.profile_replay):
            attention_step()
        torch.cuda.synchronize(device)
        print(f"profile replay complete: decode_attention x {args.profile_replay}", flush=True)
        return 0

    # -------------------------------------------------------------- timed steps
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start_evt = torch.cuda.Event(enable_timing=True)
    end_evt = torch.cuda.Event(enable_timing=True)
    start_evt.record(stream)
    for _ in range(args.steps):
        step()
    end_evt.record(stream)
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    step_ms = start_evt.elapsed_time(end_evt) / args.steps
    log(f"[bench] {args.steps} steps: {step_ms:.3f} ms/step (wall {wall_s * 1000 / args.steps:.3f})")
    # The dominant kernel on its own, at the rate it runs inside the step:
    # the same varlen gathers back to back over the 28 layers' caches, one
    # event pair around them (the host enqueues a call far faster than the
    # ~1 ms kernel runs, so the stream never idles and no per-launch
    # instrumentation is counted).
    ctx = packer.pack_decode(batch)
    plan = backend.build_gather_plan(cache[0, 0], ctx.block_tables, ctx.cu_seqlens_k, total)
    torch.cuda.synchronize()
    start_evt.record(stream)
    for _ in range(args.steps):
        for layer in range(L):
            backend.gather_varlen(cache[0, layer], cache[1, layer], ctx.block_tables, ctx.cu_seqlens_k,
                                  total, plan=plan, out=(k_out, v_out))
    end_evt.record(stream)
    torch.cuda.synchronize()
    gather_launch_us = start_evt.elapsed_time(end_evt) * 1e3 / (args.steps * L)
    log(f"[bench] gather back to back: {gather_launch_us:.1f} us per launch "
        f"(x {L} = {gather_launch_us * L / 1e3:.3f} ms of the {step_ms:.3f} ms step)")
    # Per-kernel breakdown in a pass of its own: the event pairs around each
    # launch are instrumentation, so they stay out of the timed steps above.
    timer = LaunchTimer(stream)
    store_timer = LaunchTimer(stream)
    for _ in range(args.steps):
        step(timer, store_timer)
    torch.cuda.synchronize()

    # Same step with the attention consumer instead of the gather.
    for _ in range(args.warmup):
        attention_step()
    torch.cuda.synchronize()
    start_evt.record(stream)
    for _ in range(args.steps):
        attention_step()
    end_evt.record(stream)
    torch.cuda.synchronize()
    attn_step_ms = start_evt.elapsed_time(end_evt) / args.steps
    attn_timer = LaunchTimer(stream)
    for _ in range(args.steps):
        attention_step(attn_timer)
    attn_us = attn_timer.durations_us()
    # per call at the rate it runs inside the step: back to back over the
    # 28 layers' caches, one event pair around them
    # (the plan built once per step, as an engine builds it)
    actx = packer.pack_decode(batch)
    torch.cuda.synchronize()
    start_evt.record(stream)
    for _ in range(args.steps):
        aplan = backend.build_attention_plan(cache[0, 0], actx.cu_seqlens_k, total)
        for layer in range(L):
            backend.paged_attention_decode(q, cache[0, layer], cache[1, layer], actx.block_tables,
                                           actx.cu_seqlens_k, total, softmax_scale, plan=aplan,
                                           out=attn_out)
    end_evt.record(stream)
    torch.cuda.synchronize()
    attn_mean = start_evt.elapsed_time(end_evt) * 1e3 / (args.steps * L)
    # The flash_attn_with_kvcache drop-in on the same contexts.  It takes only
    # the lengths tensor: the first call of a step reads the context total
    # back and builds the plan, which the step's other layers reuse; each
    # step here passes a new lengths tensor, as an engine's step does.
    from nanokv.flash import flash_attn_with_kvcache

    q4 = q.unsqueeze(1)
    flash_attn_with_kvcache(q4, cache[0, 0], cache[1, 0], cache_seqlens=actx.context_lens.clone(),
                            block_table=actx.block_tables, softmax_scale=softmax_scale, causal=True)
    torch.cuda.synchronize()
    step_lengths = [actx.context_lens.clone() for _ in range(args.steps)]
    torch.cuda.synchronize()
    start_evt.record(stream)
    for lengths in step_lengths:
        for layer in range(L):
            flash_attn_with_kvcache(q4, cache[0, layer], cache[1, layer], cache_seqlens=lengths,
                                    block_table=actx.block_tables, softmax_scale=softmax_scale,
                                    causal=True)
    end_evt.record(stream)
    torch.cuda.synchronize()
    flash_us = start_evt.elapsed_time(end_evt) * 1e3 / (args.steps * L)
    attn_bytes = (total * wl.num_kv_heads * wl.head_dim * 2 * q.element_size()
                  + 2 * q.numel() * q.element_size())
    log(f"[bench] {args.steps} store+attention steps: {attn_step_ms:.3f} ms/step, "
        f"attention {attn_mean:.1f} us/layer")

    store_bytes = wl.store_bytes()
    gather_bytes = wl.gather_bytes()
    step_bytes = store_bytes + gather_bytes
    gbps = step_bytes / (step_ms * 1e-3) / 1e9
    gather_launch_bytes = wl.gather_bytes(layers=1)
    gather_us = timer.durations_us()
    store_us = store_timer.durations_us()
    achieved = gather_launch_bytes / (gather_launch_us * 1e-6) / 1e9
    consistent = L * gather_launch_us <= step_ms * 1e3
    if not consistent:
        log(f"[bench] WARNING: {L} x {gather_launch_us:.1f} us of back-to-back gathers exceed the "
            f"{step_ms:.3f} ms step")
    profiled = profiled_median(PROFILE_FILE, "gather_planned_kernel", gather_launch_bytes)
    same_host = same_host_roofline(same_host_trace, gather_launch_bytes, gather_launch_us)
    same_host_frac = (round(gather_launch_bytes / (same_host["median_us"] * 1e3) / MI355X_HBM_PEAK_GBPS, 4)
                      if same_host and "median_us" in same_host else None)

    fused_step = measure_fused_step(wl, device, backend, packer, batch, cache, new_k, new_v, total,
                                    k_out, v_out, args.steps, args.warmup)
    log(f"[bench] fused store+gather step: {fused_step['ms_per_step']:.3f} ms/step "
        f"({fused_step['gbps']:.0f} GB/s of its own bytes)")

    copy_reference = measure_copy_reference(wl, device, backend, packer, cache, total, k_out, v_out,
                                            args.steps)
    log(f"[bench] copy reference: torch copy_ {copy_reference['torch_copy_gbps']:.0f} GB/s, "
        f"gather over contiguous tables {copy_reference['gather_contiguous_tables_gbps']:.0f} GB/s")

    block_pool = measure_block_pool(wl, device, packer, batch, args.steps, args.warmup)
    log(f"[bench] block pool: apply {block_pool['apply_kernel_us']:.1f} us, step "
        f"{block_pool['stream_us_per_step']:.1f} us stream / {block_pool['host_us_per_step']:.1f} us host")

    prefill_attention = None
    if args.prefill_attention and not args.profile:
        prefill_attention = measure_prefill_attention(device, backend, args.steps)
        log(f"[bench] prefill attention (chunked prefill, 8192 tokens): "
            f"{prefill_attention['us']:.1f} us, {prefill_attention['tflops']:.0f} TFLOP/s, "
            f"torch SDPA path {prefill_attention['torch_sdpa_path_us']:.0f} us")

    grouped_decode = measure_grouped_decode(device, backend, wl, args.steps)
    for rec in grouped_decode:
        log(f"[bench] decode attention {rec['layout']}: {rec['us']:.1f} us, "
            f"{rec['achieved']:.0f} GB/s ({rec['kernel']})")

    gpu_reference = None
    if args.gpu_reference and not args.profile:
        gpu_reference = {
            "what": "the reference pytorch backend's store/gather restated with its torch ops "
                    "(index_copy_ / index_select), driven as the reference's SDPA decode drives it, "
                    "on the same GPU",
            "decode_step": measure_torch_reference_step(wl, device, cache, new_k, new_v, batch,
                                                        packer, step_ms),
            "decode_step_hip_backend_unchanged_sdpa": measure_torch_reference_step(
                wl, device, cache, new_k, new_v, batch, packer, step_ms, ref=backend),
            "microbenchmark": measure_reference_matrix(device, backend),
        }
        log(f"[bench] torch reference decode step: "
            f"{gpu_reference['decode_step']['ms_per_step']:.1f} ms/step "
            f"({gpu_reference['decode_step']['speedup_of_hip']:.1f}x slower than hip); the hip "
            f"backend driven the same way: "
            f"{gpu_reference['decode_step_hip_backend_unchanged_sdpa']['ms_per_step']:.1f} ms/step")

    other_workloads = None
    if args.workload_iterations > 0 and not args.profile:
        other_workloads = measure_other_workloads(device, args.workload_iterations)
        for r in other_workloads:
            if r["gbps_at_p50"] is not None:
                log(f"[bench] {r['workload']} {r['operation']}: p50 {r['p50_us']:.2f} us, "
                    f"{r['gbps_at_p50']:.0f} GB/s")

    traffic = measured_traffic(PROFILE_FILE, "gather_planned_kernel", wl.gather_bytes(layers=1))
    attn_traffic = measured_traffic(ATTENTION_PROFILE_FILE, "attn_decode_", attn_bytes)

    cpu_baseline = None
    if not args.profile and args.cpu_baseline_layers > 0:
        check_layers = [int(x) for x in args.check_layers.split(",") if x.strip()]

        def gpu_layer(layer: int) -> dict:
            """Host copies of the GPU store+gather and attention outputs of
            one layer for the packed step, and the layer's cache before the
            store (the store is idempotent: the timed steps stored the same
            rows, so the oracle replaying it on this copy is exact)."""
            tables = wl.padded_block_tables()
            used = np.unique(tables[tables >= 0])
            index = torch.from_numpy(used.astype(np.int64)).to(device)
            kc, vc = cache[0, layer], cache[1, layer]
            before = [c.index_select(0, index).cpu().view(torch.int16).numpy() for c in (kc, vc)]
            ctx = packer.pack_decode(batch)
            plan = backend.build_gather_plan(kc, ctx.block_tables, ctx.cu_seqlens_k, total)
            backend.store(new_k[layer], new_v[layer], kc, vc, ctx.slot_mapping)
            backend.gather_varlen(kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total,
                                  plan=plan, out=(k_out, v_out))
            backend.paged_attention_decode(q, kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total,
                                           softmax_scale, out=attn_out)
            torch.cuda.synchronize()
            return {"used_blocks": used, "before": before,
                    "k_out": k_out.cpu().view(torch.int16).numpy(),
                    "v_out": v_out.cpu().view(torch.int16).numpy(),
                    "attention": attn_out.float().cpu().numpy(),
                    "q": q.float().cpu().numpy(), "scale": softmax_scale}

        cpu_baseline = cpu_baseline_leg(wl, args.cpu_baseline_layers, args.cpu_baseline_repeats,
                                        check_layers, gpu_layer,
                                        args.cpu_baseline_workloads.split(","),
                                        runs=args.cpu_baseline_runs)

    result = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "continuous-batching decode step, Qwen3-VL-2B LM KV shape",
            "layers": L,
            "live_sequences": B,
            "context_tokens": total,
            "context_law": "log-uniform [256, 16384], 16 evicted + 16 admitted",
            "kv_heads": wl.num_kv_heads,
            "head_dim": wl.head_dim,
            "block_size": wl.block_size,
            "num_blocks": wl.num_blocks,
            "cache_bytes": int(cache.numel() * cache.element_size()),
            "parallelism": "single GPU",
        },
        "hbm_fraction": round(gbps / MI355X_HBM_PEAK_GBPS, 4),
        "decode_tokens_per_s": round(B / (step_ms * 1e-3), 2),
        "settle_s": args.settle_s,
        "step_bytes": step_bytes,
        "reference_effective_bytes_per_step": L * (
            effective_bytes("store", B, wl.num_kv_heads, wl.head_dim, 2)
            + 2 * effective_bytes("gather", total, wl.num_kv_heads, wl.head_dim, 2)),
        "kernels": {
            "note": "per-launch event pairs in a pass of their own (each includes the time from "
                    "the start event to the kernel's start); the roofline uses the back-to-back rate",
            "gather_varlen_planned_us": summarize_latencies(gather_us),
            "store_us": summarize_latencies(store_us),
        },
        "roofline": {
            "kernel": "gather_planned_kernel (K+V varlen gather, one layer)",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": MI355X_HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / MI355X_HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": (str(PROFILE_FILE.relative_to(REPO_ROOT)) if traffic else None),
            "algorithmic_bytes_per_launch": gather_launch_bytes,
            "us_per_launch": round(gather_launch_us, 2),
            "timing": f"{args.steps} x {L} gathers back to back over the layers' caches, one event "
                      f"pair around them, on the stream the kernel runs on",
            "launches_per_step_us": round(L * gather_launch_us, 1),
            "within_step": consistent,
            "timing_source": "hip events around the back-to-back launches (achieved, frac, "
                             "us_per_launch); the rocprofv3 figures of the same kernel follow",
            "frac_rocprof_same_host": same_host_frac,
            "rocprof_median_us": profiled,
            "frac_rocprof_committed": (round(gather_launch_bytes / (profiled * 1e3)
                                             / MI355X_HBM_PEAK_GBPS, 4) if profiled else None),
            "rocprof_source": str(PROFILE_FILE.relative_to(REPO_ROOT)) if profiled else None,
            "rocprof_same_host": same_host,
        },
        "attention": {
            "kernel": "paged_attention_decode (split-K partials + merge, one layer, 16 q heads "
                      "over 8 kv heads, straight from the paged cache)",
            "partial_kernel": decode_kernel_name(8, 2),
            "us_bracketed": summarize_latencies(attn_us),
            "achieved": round(attn_bytes / (attn_mean * 1e-6) / 1e9, 2),
            "peak": MI355X_HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(attn_bytes / (attn_mean * 1e-6) / 1e9 / MI355X_HBM_PEAK_GBPS, 4),
            "algorithmic_bytes_per_launch": attn_bytes,
            "traffic": attn_traffic,
            "traffic_source": (str(ATTENTION_PROFILE_FILE.relative_to(REPO_ROOT))
                               if attn_traffic else None),
            "us_per_call": round(attn_mean, 2),
            "timing": "calls back to back over the layers' caches (plan built once), one event pair",
            "flash_attn_with_kvcache_us_per_call": round(flash_us, 2),
            "flash_dropin_over_direct": round(flash_us / attn_mean, 4),
            "step_ms_store_attention": round(attn_step_ms, 4),
            "decode_tokens_per_s_store_attention": round(B / (attn_step_ms * 1e-3), 2),
        },
        "fused_store_gather_step": fused_step,
        "copy_reference": copy_reference,
        "other_workloads": other_workloads,
        "prefill_attention": prefill_attention,
        "grouped_decode_attention": grouped_decode,
        "gpu_reference": gpu_reference,
        "block_pool": block_pool,
        "cpu_baseline": cpu_baseline,
        "report_schema": "nanokv.paged_kv_bench.v2",
        "identity": environment_identity(device),
    }
    print(json.dumps(result), flush=True)
    return 0


MI355X_BF16_DENSE_TFLOPS = 2500.0

# Grouped-query layouts of the Qwen vision-language families: (name, kv heads,
# query heads per kv head).  16 over 8 is the decode step's own layout.
GROUPED_LAYOUTS = (
    ("Qwen2.5-VL-3B: 16 q / 2 kv heads", 2, 8),
    ("Qwen2.5-VL-7B: 28 q / 4 kv heads", 4, 7),
    ("Qwen3-VL-8B: 32 q / 8 kv heads", 8, 4),
)


GROUPED_CASES = {"grouped_decode_2x8": (2, 8), "grouped_decode_4x7": (4, 7),
                 "grouped_decode_8x4": (8, 4)}


def grouped_decode_setup(device, backend, wl, hkv: int, group: int, gen) -> dict:
    """One decode-attention layer over the decode step's 256 contexts (block
    256, blocks placed at random by ``gen``) with ``hkv`` kv heads and
    ``group`` query heads per kv head: caches, tables, q, plan and the call.
    Bytes = the K and V rows read once, plus q and out."""
    import numpy as np
    import torch

    lens = np.asarray(wl.num_tokens, dtype=np.int64)
    bs = wl.block_size
    need = -(-lens // bs)
    nb = int(need.sum()) + 8
    total = int(lens.sum())
    perm = torch.randperm(nb, device=device, generator=gen).to(torch.int32)
    tables = torch.full((lens.size, int(need.max())), -1, dtype=torch.int32, device=device)
    cursor = 0
    for i, n in enumerate(need.tolist()):
        tables[i, :n] = perm[cursor:cursor + n]
        cursor += n
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=device)
    kc = torch.empty((nb, bs, hkv, 128), dtype=torch.bfloat16, device=device).normal_(generator=gen)
    vc = torch.empty_like(kc).normal_(generator=gen)
    q = torch.randn((lens.size, hkv * group, 128), device=device, generator=gen).to(torch.bfloat16)
    out = torch.empty_like(q)
    plan = backend.build_attention_plan(kc, cu, total)
    scale = 1.0 / math.sqrt(128)

    def call():
        backend.paged_attention_decode(q, kc, vc, tables, cu, total, scale, plan=plan, out=out)

    return {"call": call, "q": q, "kc": kc, "vc": vc, "tables": tables, "lens": lens, "out": out,
            "scale": scale, "bytes": total * hkv * 128 * 2 * 2 + 2 * q.numel() * 2}


def host_attention(q, k, v, scale: float, offset: int | None = None):
    """float32 softmax(scale q K^T) V on the host for one request: q [Lq,
    Hq, D], k / v [Lk, Hkv, D]; query head h reads kv head h // (Hq / Hkv);
    with ``offset``, query j sees keys [0, offset + j] (bottom-right causal)."""
    import torch

    group = q.shape[1] // k.shape[1]
    keys = k.float().cpu().repeat_interleave(group, dim=1).transpose(0, 1)      # [Hq, Lk, D]
    values = v.float().cpu().repeat_interleave(group, dim=1).transpose(0, 1)
    queries = q.float().cpu().transpose(0, 1)                                    # [Hq, Lq, D]
    scores = torch.matmul(queries, keys.transpose(1, 2).contiguous()) * scale    # [Hq, Lq, Lk]
    if offset is not None:
        lq, lk = q.shape[0], k.shape[0]
        visible = torch.arange(lk)[None, :] <= (torch.arange(lq) + offset)[:, None]
        scores = scores.masked_fill(~visible[None], float("-inf"))
    return torch.matmul(torch.softmax(scores, dim=-1), values).transpose(0, 1)   # [Lq, Hq, D]


def attention_tolerance(ref, ref_abs):
    """Allowed error of a decode-attention output: 1e-3 + 2^-8 (|ref| +
    ref_abs), ref_abs being the same attention over |V|.  The MFMA kernel
    rounds its softmax weights to the input type (as flash attention does),
    so an output near zero by cancellation carries the error of its terms;
    the same bound holds the GPU tests."""
    return 1e-3 + 2.0 ** -8 * (abs(ref) + ref_abs)


def check_decode_attention(backend, case: dict, sample: int = 6) -> None:
    """The decode attention of ``sample`` sequences against host_attention
    over their K/V rows gathered bit-exactly, within attention_tolerance."""
    import numpy as np
    import torch

    case["call"]()
    torch.cuda.synchronize()
    for i in np.linspace(0, len(case["lens"]) - 1, sample).astype(int).tolist():
        n = int(case["lens"][i])
        table = case["tables"][i, : -(-n // case["kc"].shape[1])].contiguous()
        keys, values = backend.gather(case["kc"], table, n), backend.gather(case["vc"], table, n)
        expect = host_attention(case["q"][i:i + 1], keys, values, case["scale"])[0]
        expect_abs = host_attention(case["q"][i:i + 1], keys, values.abs(), case["scale"])[0]
        err = (case["out"][i].float().cpu() - expect).abs()
        if bool((err > attention_tolerance(expect, expect_abs)).any()):
            raise AssertionError(f"decode attention, sequence {i}: max error {float(err.max()):.3e}")


def decode_kernel_name(kv_heads: int, group: int) -> str:
    """The kernel nkv_paged_attention_decode runs for a head layout: the
    range split below 8 kv heads, the entry split from 8 on (any group of
    up to 16 query heads per kv head)."""
    return "attn_decode_entry_kernel" if kv_heads >= 8 else "attn_decode_range_kernel"


def measure_grouped_decode(device, backend, wl, reps: int) -> list[dict]:
    """Paged-attention decode of one layer over the decode step's 256
    contexts for the grouped-query layouts above (the MFMA decode kernel).
    One event pair on the current stream around `reps` calls (partials +
    merge)."""
    import torch

    from nanokv.benchmark import MI355X_HBM_PEAK_GBPS

    gen = torch.Generator(device=device).manual_seed(29)
    records = []
    for name, hkv, g in GROUPED_LAYOUTS:
        case = grouped_decode_setup(device, backend, wl, hkv, g, gen)
        for _ in range(3):
            case["call"]()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            case["call"]()
        end.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(end) * 1e3 / reps
        achieved = case["bytes"] / (us * 1e-6) / 1e9
        records.append({
            "layout": name, "kv_heads": hkv, "q_heads_per_kv_head": g,
            "kernel": decode_kernel_name(hkv, g),
            "us": round(us, 2), "algorithmic_bytes": case["bytes"], "achieved": round(achieved, 1),
            "unit": "GB/s", "frac": round(achieved / MI355X_HBM_PEAK_GBPS, 4),
        })
        del case
        torch.cuda.empty_cache()
    return records


def chunked_prefill_shape(seed: int = 17):
    """16 requests in one 8192-token chunk, lengths uniform in [128, 4096]
    scaled to the chunk; requests 0-7 continue after 1-4 cached 256-row
    blocks.  Returns (query lengths, context lengths)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    raw = rng.integers(128, 4097, 16).astype(np.float64)
    q_lens = np.floor(raw / raw.sum() * 8192).astype(np.int64)
    q_lens[-1] += 8192 - q_lens.sum()
    cached = np.zeros(16, np.int64)
    cached[:8] = rng.integers(1, 5, 8) * 256
    return q_lens.tolist(), (q_lens + cached).tolist()


def prefill_setup(device, backend) -> dict:
    """The chunked-prefill step's paged prefill attention: Qwen3-VL-2B's 16
    query heads over 8 kv heads, 256-row blocks placed at random; caches,
    tables, q, plan and the call.  Algorithmic FLOPs = 4 x head_dim x query
    heads x the (query, visible key) pairs."""
    import numpy as np
    import torch

    q_lens, k_lens = chunked_prefill_shape()
    hkv, g, bs, dim = 8, 2, 256, 128
    need = [-(-k // bs) for k in k_lens]
    nb = sum(need) + 4
    gen = torch.Generator(device=device).manual_seed(19)
    kc = torch.randn((nb, bs, hkv, dim), device=device, generator=gen).to(torch.bfloat16)
    vc = torch.randn_like(kc)
    perm = torch.randperm(nb, device=device, generator=gen).to(torch.int32)
    tables = torch.full((len(q_lens), max(need)), -1, dtype=torch.int32, device=device)
    offset = 0
    for i, n in enumerate(need):
        tables[i, :n] = perm[offset:offset + n]
        offset += n
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32, device=device)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(k_lens)]), dtype=torch.int32, device=device)
    q = torch.randn((sum(q_lens), hkv * g, dim), device=device, generator=gen).to(torch.bfloat16)
    scale = 1.0 / math.sqrt(dim)
    plan = backend.build_prefill_plan(q, kc, cu_q, cu_k)
    out = torch.empty_like(q)

    def call():
        backend.paged_attention_prefill(q, kc, vc, tables, cu_q, cu_k, scale, plan=plan, out=out)

    pairs = sum(sum(lk - lq + j + 1 for j in range(lq)) for lq, lk in zip(q_lens, k_lens))
    return {"call": call, "q": q, "kc": kc, "vc": vc, "tables": tables, "cu_q": cu_q, "cu_k": cu_k,
            "q_lens": q_lens, "k_lens": k_lens, "scale": scale, "out": out,
            "flops": 4 * dim * hkv * g * pairs, "dims": (hkv, g, dim)}


def check_prefill_attention(backend, case: dict, requests: int = 2) -> None:
    """The prefill attention of the ``requests`` shortest requests against
    host_attention (bottom-right causal) over their K/V rows gathered
    bit-exactly, within 1e-3 + 2^-7 (|ref| + the same attention over |V|):
    twice the bound of the parity tests, whose terms are the bf16 weights,
    the output rounding and accumulation order."""
    import torch

    case["call"]()
    torch.cuda.synchronize()
    starts = case["cu_q"].cpu().tolist()
    order = sorted(range(len(case["q_lens"])), key=lambda i: case["k_lens"][i])[:requests]
    for i in order:
        lq, lk = case["q_lens"][i], case["k_lens"][i]
        table = case["tables"][i, : -(-lk // case["kc"].shape[1])].contiguous()
        k = backend.gather(case["kc"], table, lk)
        v = backend.gather(case["vc"], table, lk)
        q = case["q"][starts[i]:starts[i] + lq]
        expect = host_attention(q, k, v, case["scale"], offset=lk - lq)
        ref_abs = host_attention(q, k, v.abs(), case["scale"], offset=lk - lq)
        err = (case["out"][starts[i]:starts[i] + lq].float().cpu() - expect).abs()
        if bool((err > 1e-3 + 2.0 ** -7 * (expect.abs() + ref_abs)).any()):
            raise AssertionError(f"prefill attention, request {i}: max error {float(err.max()):.3e}")


def measure_prefill_attention(device, backend, reps: int) -> dict:
    """Causal prefill attention read straight from the paged cache (the
    Flash path's prefill call) on the chunked-prefill step
    (:func:`prefill_setup`).  Beside it, the reference's SDPA prefill on the
    same GPU: per request, the pytorch-backend gathers of K and V and SDPA
    with the prefix-causal mask (nanovllm/layers/attention.py:226-282)."""
    import torch

    from nanokv.benchmark import LaunchTimer

    case = prefill_setup(device, backend)
    q_lens, k_lens, q, kc, vc, tables = (case[k] for k in ("q_lens", "k_lens", "q", "kc", "vc", "tables"))
    cu_q, scale, flops = case["cu_q"], case["scale"], case["flops"]
    stream = torch.cuda.current_stream(device)
    timer = LaunchTimer(stream)
    for _ in range(3):
        case["call"]()
    torch.cuda.synchronize()
    # One event pair around back-to-back launches: the host enqueues a call
    # faster than the kernel runs, so the stream never idles and the mean is
    # the kernel's duration (per-launch pairs would also count the time the
    # idle stream waits for the host's next call).
    t0 = timer.start()
    for _ in range(reps):
        case["call"]()
    timer.stop(t0)
    us = timer.durations_us()[0] / reps
    ref = reference_backend()

    def sdpa_path():
        for i, (lq, lk) in enumerate(zip(q_lens, k_lens)):
            k = ref.gather(kc, tables[i], lk)
            v = ref.gather(vc, tables[i], lk)
            query = q[int(cu_q[i]):int(cu_q[i + 1])]
            visible = (torch.arange(lk, device=device)[None, :]
                       <= (torch.arange(lq, device=device) + (lk - lq))[:, None])
            torch.nn.functional.scaled_dot_product_attention(
                query.transpose(0, 1).unsqueeze(0), k.transpose(0, 1).unsqueeze(0).contiguous(),
                v.transpose(0, 1).unsqueeze(0).contiguous(), attn_mask=visible[None, None],
                scale=scale, enable_gqa=True)

    sdpa_path()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(3):
        sdpa_path()
    torch.cuda.synchronize()
    sdpa_us = (time.perf_counter() - t0) / 3 * 1e6
    return {
        "workload": "chunked prefill: 16 requests, 8192 query tokens, 8 continuing after 1-4 "
                    "cached blocks; 16 query heads over 8 kv heads, head_dim 128, 256-row blocks",
        "kernel": "attn_prefill_kernel<2> (MFMA 16x16x32 bf16, causal, paged)",
        "us": round(us, 2),
        "algorithmic_flops": flops,
        "tflops": round(flops / us / 1e6, 1),
        "peak_tflops": MI355X_BF16_DENSE_TFLOPS,
        "frac": round(flops / us / 1e6 / MI355X_BF16_DENSE_TFLOPS, 4),
        "bound": "mfma",
        "torch_sdpa_path_us": round(sdpa_us, 1),
        "speedup_vs_torch_sdpa_path": round(sdpa_us / us, 2),
    }


OTHER_WORKLOADS = ("decode_store", "chunked_prefill", "prefix_gather", "narrow_rows")


def measure_other_workloads(device, iterations: int) -> list[dict]:
    """The single-layer store / gather configurations of the paged-KV
    micro-benchmark (decode store, chunked-prefill store, prefix-cache
    gather, narrow rows), each on its own cache, checked bit-exactly against
    the reference backend's torch ops first.  Two timings per operation:
    p50 of per-launch event pairs with the MALL evicted by a 512 MiB read
    before every launch (the reference benchmark's per-iteration method),
    and the steady-state rate of launches back to back over 16 rotating
    disjoint input/output sets (write-backs of earlier launches included).
    One compact record per operation that moves bytes."""
    import torch

    from nanokv.benchmark import run_workload

    records = []
    for name in OTHER_WORKLOADS:
        for r in run_workload(name, iterations=iterations, warmup=5, device=device):
            if r["algorithmic_bytes"] == 0:
                continue
            records.append({
                "workload": name, "operation": r["operation"],
                "algorithmic_bytes": r["algorithmic_bytes"],
                "p50_us": round(r["latency"]["p50_us"], 2),
                "gbps_at_p50": r["gbps_at_p50"], "hbm_fraction": r["hbm_fraction"],
                "steady_state": r.get("steady_state"),
            })
        torch.cuda.empty_cache()
    return records


def measure_fused_step(wl, device, backend, packer, batch, cache, new_k, new_v, total, k_out, v_out,
                       steps: int, warmup: int) -> dict:
    """The same decode step with each layer's store and gather as one fused
    launch (nkv_store_gather: each sequence's one new token is the last row
    of its context, read once and written to the cache and the output).
    Layer 0's outputs are first compared bit-exactly with the separate
    store-then-gather path's.  Bytes are the fused launch's own: the store's
    and the gather's, less the new rows the gather would read back."""
    import torch

    B, L = wl.num_seqs, wl.num_layers
    cu_q = torch.arange(B + 1, dtype=torch.int32, device=device)
    ctx = packer.pack_decode(batch)
    plan = backend.build_gather_plan(cache[0, 0], ctx.block_tables, ctx.cu_seqlens_k, total)
    backend.store(new_k[0], new_v[0], cache[0, 0], cache[1, 0], ctx.slot_mapping)
    backend.gather_varlen(cache[0, 0], cache[1, 0], ctx.block_tables, ctx.cu_seqlens_k, total,
                          plan=plan, out=(k_out, v_out))
    fk, fv = torch.empty_like(k_out), torch.empty_like(v_out)

    def step(out=(fk, fv)):
        c = packer.pack_decode(batch)
        sg_plan = backend.build_store_gather_plan(cache[0, 0], c.block_tables, cu_q, c.cu_seqlens_k,
                                                  B, total)
        for layer in range(L):
            backend.store_gather(new_k[layer], new_v[layer], cache[0, layer], cache[1, layer],
                                 c.slot_mapping, c.block_tables, cu_q, c.cu_seqlens_k, total,
                                 plan=sg_plan, out=out)

    step()
    torch.cuda.synchronize()
    # layers > 0 overwrote fk/fv; redo layer 0 alone for the comparison
    c = packer.pack_decode(batch)
    sg_plan = backend.build_store_gather_plan(cache[0, 0], c.block_tables, cu_q, c.cu_seqlens_k, B, total)
    backend.store_gather(new_k[0], new_v[0], cache[0, 0], cache[1, 0], c.slot_mapping, c.block_tables,
                         cu_q, c.cu_seqlens_k, total, plan=sg_plan, out=(fk, fv))
    torch.cuda.synchronize()
    if not (torch.equal(fk.view(torch.int16), k_out.view(torch.int16))
            and torch.equal(fv.view(torch.int16), v_out.view(torch.int16))):
        raise AssertionError("fused store+gather differs from store then gather on layer 0")
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    step_bytes = L * (wl.store_bytes(layers=1) + wl.gather_bytes(layers=1)
                      - int((wl.slot_mapping >= 0).sum()) * 2 * wl.row_bytes)
    return {
        "what": "pack + store+gather plan + 28 x nkv_store_gather (one launch per layer); "
                "layer 0 bit-identical to store then gather",
        "ms_per_step": round(ms, 4),
        "decode_tokens_per_s": round(B / (ms * 1e-3), 2),
        "algorithmic_bytes_per_step": step_bytes,
        "gbps": round(step_bytes / (ms * 1e-3) / 1e9, 2),
    }


def measure_copy_reference(wl, device, backend, packer, cache, total, k_out, v_out, reps: int) -> dict:
    """Context for the gather's roofline fraction, on the same payload (one
    layer's K and V contexts, read once and written once):
    - the runtime's plain device-to-device copy (torch ``copy_``) of a
      contiguous buffer of that size;
    - the gather itself over block tables that place every sequence's blocks
      back to back in the cache, so only the block-table indirection differs
      from the copy of contiguous memory."""
    import numpy as np
    import torch

    from nanokv.benchmark import LaunchTimer
    from nanokv.packing import SequenceBatch

    stream = torch.cuda.current_stream(device)
    payload = 2 * k_out.numel() * k_out.element_size()
    src = torch.ones(payload // 2, dtype=torch.int16, device=device)
    dst = torch.empty_like(src)
    copy_timer = LaunchTimer(stream)
    for i in range(reps + 2):
        t0 = copy_timer.start() if i >= 2 else None
        dst.copy_(src)
        if t0 is not None:
            copy_timer.stop(t0)
    copy_us = copy_timer.durations_us()
    del src, dst

    counts = -(-wl.num_tokens.astype(np.int64) // wl.block_size)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    if offsets[-1] > wl.num_blocks:
        raise RuntimeError("the contiguous layout needs more blocks than the cache holds")
    batch = SequenceBatch(wl.num_tokens, offsets, np.arange(offsets[-1]))
    ctx = packer.pack_decode(batch)
    kc, vc = cache[0, 0], cache[1, 0]
    plan = backend.build_gather_plan(kc, ctx.block_tables, ctx.cu_seqlens_k, total)
    gather_timer = LaunchTimer(stream)
    for i in range(reps + 2):
        t0 = gather_timer.start() if i >= 2 else None
        backend.gather_varlen(kc, vc, ctx.block_tables, ctx.cu_seqlens_k, total,
                              plan=plan, out=(k_out, v_out))
        if t0 is not None:
            gather_timer.stop(t0)
    gather_us = gather_timer.durations_us()
    torch.cuda.synchronize()
    copy_mean = float(np.mean(copy_us))
    gather_mean = float(np.mean(gather_us))
    return {
        "payload_bytes": payload,
        "torch_copy_us": round(copy_mean, 2),
        "torch_copy_gbps": round(2 * payload / (copy_mean * 1e-6) / 1e9, 2),
        "gather_contiguous_tables_us": round(gather_mean, 2),
        "gather_contiguous_tables_gbps": round(wl.gather_bytes(layers=1) / (gather_mean * 1e-6) / 1e9, 2),
        "note": "bytes counted as read + write of the payload; the gather's figure uses its "
                "algorithmic bytes (payload read + written, plus block ids)",
    }


def block_pool_steps(wl, seed: int = 11):
    """The decode step's block bookkeeping as an endless run of scheduler
    steps: the 256 running sequences each grow by one token (a new block
    when the token opens one), then 16 finish and 16 are admitted with
    contexts from the same law.  Yields, per step, the op list and the
    running (slot, tokens) pairs; block accounting is exact on the host
    because no block is shared."""
    import numpy as np

    rng = np.random.default_rng(seed)
    bs = wl.block_size
    lens = {slot: int(n) for slot, n in enumerate(wl.num_tokens)}
    free_slots = list(range(wl.num_seqs, 2 * wl.num_seqs))
    held = {slot: -(-n // bs) for slot, n in lens.items()}
    free_blocks = wl.num_blocks - sum(held.values())
    yield [("allocate", slot, held[slot]) for slot in lens], dict(lens)
    while True:
        ops = []
        for slot in list(lens):
            if lens[slot] % bs == 0:
                if free_blocks == 0:  # can_append fails: the sequence waits
                    continue
                ops.append(("append", slot))
                held[slot] += 1
                free_blocks -= 1
            lens[slot] += 1
        for slot in rng.choice(sorted(lens), 16, replace=False).tolist():
            ops.append(("deallocate", slot))
            free_blocks += held.pop(slot)
            del lens[slot]
            free_slots.append(slot)
        contexts = np.floor(np.exp(np.log(256) + rng.random(16) * (np.log(16384) - np.log(256))))
        for n_tokens in contexts.astype(np.int64).tolist():
            n = -(-int(n_tokens) // bs)
            if n > free_blocks or not free_slots:
                continue
            slot = free_slots.pop(0)
            ops.append(("allocate", slot, n))
            held[slot] = n
            free_blocks -= n
            lens[slot] = int(n_tokens)
        yield ops, dict(lens)


def replay_block_pool(wl, device, packer, steps: int) -> None:
    """The profiling replay of the block pool: the admission of the decode
    step's sequences, then ``steps`` scheduler steps (each flushed to the
    device pool and packed from it), with no events.  Checked: no op failed,
    and the pool's free count equals its blocks less those the steps hold
    (block_pool_steps tracks them exactly; no block is shared)."""
    import torch

    from nanokv.pool import DeviceBlockPool

    width = -(-(16384 + 4 * steps + 1) // wl.block_size) + 1
    pool = DeviceBlockPool(wl.num_blocks, wl.block_size, max_seqs=2 * wl.num_seqs,
                           max_blocks_per_seq=width, device=device)
    held = 0
    for k, (ops, lens) in enumerate(block_pool_steps(wl)):
        if k > steps:
            break
        for op in ops:
            if op[0] == "append":
                pool.append(op[1])
            elif op[0] == "deallocate":
                pool.deallocate(op[1])
            else:
                pool.allocate(op[1], op[2])
        pool.flush()
        slots = sorted(lens)
        packer.pack_decode_pool(pool, slots, [lens[s] for s in slots])
        held = sum(-(-n // wl.block_size) for n in lens.values())
    torch.cuda.synchronize(device)
    pool.check()
    live = int(pool.meta[2].item())
    if live != wl.num_blocks - held:
        raise AssertionError(f"block pool holds {wl.num_blocks - live} blocks, the steps {held}")


def measure_block_pool(wl, device, packer, batch, steps: int, warmup: int) -> dict:
    """Per decode step: record the step's BlockManager calls, replay them
    on the device pool and pack the step from the pool's tables, against
    packing the same batch shape from an uploaded CSR (the path without
    the pool).  GPU time from events on the current stream; host time is
    the Python recording + launch cost."""
    import numpy as np
    import torch

    from nanokv.benchmark import LaunchTimer
    from nanokv.pool import DeviceBlockPool

    width = -(-(16384 + 4 * (steps + warmup) + 1) // wl.block_size) + 1
    pool = DeviceBlockPool(wl.num_blocks, wl.block_size, max_seqs=2 * wl.num_seqs,
                           max_blocks_per_seq=width, device=device)
    stream = torch.cuda.current_stream(device)
    gen = block_pool_steps(wl)
    pool_timer, csr_timer, apply_timer = LaunchTimer(stream), LaunchTimer(stream), LaunchTimer(stream)
    host_s, log_bytes = [], []

    def run(ops, lens, timed: bool):
        t0 = time.perf_counter()
        e0 = pool_timer.start() if timed else None
        for op in ops:
            if op[0] == "append":
                pool.append(op[1])
            elif op[0] == "deallocate":
                pool.deallocate(op[1])
            else:
                pool.allocate(op[1], op[2])
        n_ops, n_args = pool.pending_ops, len(pool._args)
        pool.flush(apply_timer if timed else None)
        slots = sorted(lens)
        packer.pack_decode_pool(pool, slots, [lens[s] for s in slots])
        if timed:
            pool_timer.stop(e0)
            host_s.append(time.perf_counter() - t0)
            log_bytes.append(16 * n_ops + 4 * n_args + 8 * len(slots))
            e1 = csr_timer.start()
            packer.pack_decode(batch)
            csr_timer.stop(e1)

    ops, lens = next(gen)
    run(ops, lens, False)
    for _ in range(warmup):
        run(*next(gen), False)
    for _ in range(steps):
        run(*next(gen), True)
    torch.cuda.synchronize()
    pool.check()
    pool_us = pool_timer.durations_us()
    csr_us = csr_timer.durations_us()
    apply_us = apply_timer.durations_us()
    csr_bytes = 4 * (2 * batch.num_seqs + 1 + int(batch.block_ids.size))
    return {
        "step": "256 running sequences +1 token (append when a block opens), 16 finish, "
                "16 admitted; replay on the device pool, then pack_decode_pool",
        "apply_kernel_us": round(float(np.mean(apply_us)), 2),
        "stream_us_per_step": round(float(np.mean(pool_us)), 2),
        "host_us_per_step": round(1e6 * float(np.mean(host_s)), 2),
        "upload_bytes_per_step": int(np.mean(log_bytes)),
        "csr_pack_stream_us_per_step": round(float(np.mean(csr_us)), 2),
        "csr_upload_bytes_per_step": csr_bytes,
        "note": "stream_us brackets the whole step with events, so it includes the host's "
                "launch gaps; apply_kernel_us brackets the apply kernel alone",
    }


def measure_torch_reference_step(wl, device, cache, new_k, new_v, batch, packer,
                                 hip_step_ms: float, steps: int = 2, ref=None) -> dict:
    """The decode step's data path as the reference's SDPA decode drives its
    backend (nanovllm/layers/attention.py:75-93, 284-300): per layer one
    store, then per sequence a host read of its context length and one
    gather each of K and V.  The packed metadata is the same as the hip
    step's (packed once, outside the timed region; the reference packs on
    the host).  The outputs are dropped where SDPA would consume them.
    ``ref`` is the backend driven (default: the torch restatement of the
    reference pytorch backend; the hip backend gives the step that switching
    paged_kv_backend alone, with SDPA unchanged, would run)."""
    import torch

    ref = ref if ref is not None else reference_backend()
    ctx = packer.pack_decode(batch)
    torch.cuda.synchronize()

    def step():
        for layer in range(wl.num_layers):
            kc, vc = cache[0, layer], cache[1, layer]
            ref.store(new_k[layer], new_v[layer], kc, vc, ctx.slot_mapping)
            for i in range(wl.num_seqs):
                n = int(ctx.context_lens[i])
                ref.gather(kc, ctx.block_tables[i], n)
                ref.gather(vc, ctx.block_tables[i], n)

    step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return {
        "ms_per_step": round(ms, 2),
        "decode_tokens_per_s": round(wl.num_seqs / (ms * 1e-3), 2),
        "store_gather_gbps": round((wl.store_bytes() + wl.gather_bytes()) / (ms * 1e-3) / 1e9, 2),
        "speedup_of_hip": round(ms / hip_step_ms, 2),
        "steps": steps,
        "timing": "host wall clock over whole steps (the per-sequence length reads synchronize)",
    }


REFERENCE_MATRIX = {  # bench_paged_kv.py's defaults in the reference
    "operations": ("store", "gather"), "dtypes": ("float16", "bfloat16"), "tokens": (1, 8, 257),
    "kv_shapes": ((1, 64), (2, 128), (8, 128)), "num_blocks": 64, "block_size": 16,
    "mapping": "random_with_skips", "seed": 17, "warmup": 100, "iterations": 1000,
}


def measure_reference_matrix(device, backend=None, iterations: int | None = None) -> dict:
    """The reference's store/gather micro-benchmark matrix with its defaults
    (bench_paged_kv.py:58-148), run by nanokv.microbench for the hip backend
    and for the reference's torch ops: per case a cache of 64 blocks of 16
    slots, K/V from N(0,1), slots a random permutation of the cache with
    every 11th slot -1, a random block table; a bit-exact gate against the
    reference's torch ops, then the p50 of per-call event timings.  Effective
    bytes are the reference's (payload x 4 for store, x 2 for gather)."""
    import numpy as np

    from nanokv import microbench as mb

    m = REFERENCE_MATRIX
    iterations = iterations or m["iterations"]
    cases = mb.expand_matrix(backends=("hip", "pytorch"), operations=m["operations"],
                             dtypes=tuple(mb.DTYPES[n] for n in m["dtypes"]),
                             token_counts=m["tokens"], kv_shapes=m["kv_shapes"],
                             block_size=m["block_size"], num_blocks=m["num_blocks"],
                             mapping=m["mapping"], seed=m["seed"])
    by_case: dict[str, dict] = {}
    for case in cases:
        result = mb.run_case(case, warmup=m["warmup"], iterations=iterations, device=device)
        key = case.selector.split(";", 1)[1]  # the selector without its backend
        record = by_case.setdefault(key, {
            "operation": case.operation, "dtype": mb.DTYPE_NAMES[case.dtype],
            "tokens": case.num_tokens, "kv_shape": f"{case.num_kv_heads}x{case.head_dim}",
            "effective_bytes": result["effective_bytes"]})
        name = "hip" if case.backend == "hip" else "torch_reference"
        record[f"{name}_p50_us"] = round(result["latency"]["p50_us"], 3)
        record[f"{name}_gbps"] = round(result["effective_gbps_at_p50"], 3)
    records = list(by_case.values())
    ratios = [r["torch_reference_p50_us"] / r["hip_p50_us"] for r in records]
    return {"cases": records, "geomean_speedup_of_hip": round(float(np.exp(np.mean(np.log(ratios)))), 3),
            "iterations": iterations, "warmup": m["warmup"], "runner": "nanokv.microbench",
            "schema_of_full_reports": mb.SCHEMA}


def cpu_baseline_leg(wl, layers: int, repeats: int, check_layers, gpu_layer,
                     workload_names, runs: int = 5) -> dict:
    """The CPU leg: the oracle checks the GPU's outputs of ``check_layers``
    (store+gather bit-exact; attention within attention_tolerance of the fp32
    oracle on 32 sequences); then the reference pytorch backend's torch ops
    are timed on host tensors (:func:`cpu_reference_baseline`, the figure
    the line reports), and the oracle's OpenMP C restatement beside them
    (:func:`openmp_port_baseline`)."""
    import numpy as np
    import torch

    from oracle import c_oracle
    from oracle import paged_kv as oracle

    threads = c_oracle.default_threads()
    tables = wl.padded_block_tables()
    cu = wl.cu_seqlens_k()
    checked = []
    for layer in check_layers:
        got = gpu_layer(layer)
        used = got["used_blocks"]
        remap = np.full(wl.num_blocks, -1, np.int64)
        remap[used] = np.arange(used.size)
        ctables = np.where(tables >= 0, remap[np.maximum(tables, 0)], -1).astype(np.int32)
        cslots = (remap[wl.slot_mapping // wl.block_size] * wl.block_size
                  + wl.slot_mapping % wl.block_size).astype(np.int32)
        hk, hv = got["before"]
        c_oracle.store(wl.key[layer].view(torch.int16).numpy(), wl.value[layer].view(torch.int16).numpy(),
                       hk, hv, cslots, threads=threads)
        for name, host in (("k_out", hk), ("v_out", hv)):
            expected = c_oracle.gather_varlen(host, ctables, cu, threads=threads)
            if not np.array_equal(got[name], expected):
                raise AssertionError(f"decode step layer {layer}: gather differs from the oracle")
        sample = np.linspace(0, wl.num_seqs - 1, 32).astype(np.int64)
        ref = oracle.paged_attention_decode(got["q"][sample], hk, hv, ctables[sample],
                                            wl.num_tokens[sample], got["scale"])
        ref_abs = oracle.paged_attention_decode(got["q"][sample], hk, hv & np.int16(0x7FFF),
                                                ctables[sample], wl.num_tokens[sample], got["scale"])
        err = np.abs(got["attention"][sample] - ref)
        if (err > attention_tolerance(ref, ref_abs)).any():
            raise AssertionError(f"decode step layer {layer}: attention differs from the oracle "
                                 f"(max err {err.max():.3e})")
        log(f"[bench] layer {layer}: store+gather bit-exact, attention max err {err.max():.2e} vs oracle")
        checked.append(layer)
    result = cpu_reference_baseline(wl, layers, workload_names, runs=runs)
    result["checked_layers"] = checked
    result["openmp_port"] = openmp_port_baseline(wl, wl.num_layers, repeats)

    # The block bookkeeping of the same decode steps on the host: the
    # oracle's restatement of BlockManager, one Python call per op as the
    # reference makes them.
    from oracle.block_pool import BlockPoolOracle

    book = BlockPoolOracle(wl.num_blocks)
    gen = block_pool_steps(wl)
    step_s = []
    for k in range(1 + 50):
        ops, _ = next(gen)
        t0 = time.perf_counter()
        for op in ops:
            if op[0] == "append":
                book.append(op[1])
            elif op[0] == "deallocate":
                book.deallocate(op[1])
            else:
                book.allocate(op[1], op[2])
        if k:
            step_s.append(time.perf_counter() - t0)
    result["block_pool_python_us_per_step"] = round(1e6 * sum(step_s) / len(step_s), 2)
    return result


def _host_cache(shape, dtype):
    """A host cache tensor with every page touched (the values never
    influence the data movement)."""
    import torch

    cache = torch.empty(shape, dtype=dtype)
    cache.view(torch.int16 if cache.element_size() == 2 else torch.int32).fill_(0x3F80)
    return cache


def _median_seconds(fn, *, min_runs: int = 3, budget_s: float = 2.0) -> tuple[float, int]:
    """Median wall time of ``fn`` over at least ``min_runs`` runs, more while
    the budget lasts (one untimed run first)."""
    fn()
    times = []
    spent = 0.0
    while len(times) < min_runs or spent < budget_s:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        spent += times[-1]
        if len(times) >= 50:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_reference_baseline(wl, layers: int, workload_names, runs: int = 5) -> dict:
    """The reference's own CPU path: the ``pytorch`` backend's torch ops
    (index_copy_ store, index_select gather of whole blocks,
    nanovllm/layers/paged_kv/pytorch_backend.py:26-50, with the validators
    that check index values on host tensors, base.py:68-72) on host tensors,
    driven as SDPAAttention drives them (one store per layer, one gather per
    sequence and per K/V, attention.py:75-93, 284-300), with
    torch.set_num_threads(the host cores this job may use).

    The decode step is sampled: ``layers`` layers (each with its own new
    rows) against ONE layer-sized host cache (the 28-layer cache does not fit
    host memory), bytes counted as on the GPU, run ``runs`` times; the median
    run's per-layer time scales to the 28-layer step.  The single-layer configurations are timed whole, each
    operation as the median of at least 3 runs."""
    import numpy as np
    import torch

    from nanokv import workloads
    from nanokv.benchmark import TorchReferenceBackend, cpu_model, host_threads

    threads = host_threads()
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    ref = TorchReferenceBackend()
    try:
        shape = (wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim)
        kc, vc = _host_cache(shape, wl.dtype), _host_cache(shape, wl.dtype)
        tables = torch.from_numpy(wl.padded_block_tables())
        slots = torch.from_numpy(wl.slot_mapping)
        lens = [int(n) for n in wl.num_tokens]

        def layer(index: int) -> None:
            ref.store(wl.key[index], wl.value[index], kc, vc, slots)
            for i, n in enumerate(lens):
                ref.gather(kc, tables[i], n)
                ref.gather(vc, tables[i], n)

        layer(0)
        run_s = []
        for _ in range(max(1, runs)):
            t0 = time.perf_counter()
            for index in range(layers):
                layer(index % wl.num_layers)
            run_s.append((time.perf_counter() - t0) / layers)
        per_layer = sorted(run_s)[len(run_s) // 2]
        layer_bytes = wl.store_bytes(layers=1) + wl.gather_bytes(layers=1)
        del kc, vc
        configs = {}
        for name in [n for n in workload_names if n]:
            w = workloads.build(name)
            wshape = (w.num_blocks, w.block_size, w.num_kv_heads, w.head_dim)
            wk, wv = _host_cache(wshape, w.dtype), _host_cache(wshape, w.dtype)
            record = {}
            if w.slot_mapping is not None:
                wslots = torch.from_numpy(w.slot_mapping)
                sec, runs = _median_seconds(lambda: ref.store(w.key, w.value, wk, wv, wslots))
                nbytes = w.store_bytes(layers=1)
                record["store"] = {"seconds": round(sec, 6), "runs": runs, "algorithmic_bytes": nbytes,
                                   "gbps": round(nbytes / sec / 1e9, 3)}
            if name != "decode_store":
                wtables = torch.from_numpy(w.padded_block_tables())
                wlens = [int(n) for n in w.context_lens]

                def gathers():
                    for i, n in enumerate(wlens):
                        ref.gather(wk, wtables[i], n)
                        ref.gather(wv, wtables[i], n)

                sec, runs = _median_seconds(gathers)
                nbytes = w.gather_bytes(layers=1)
                record["gather_kv"] = {"seconds": round(sec, 6), "runs": runs, "algorithmic_bytes": nbytes,
                                       "gbps": round(nbytes / sec / 1e9, 3)}
            configs[name] = record
            del wk, wv
    finally:
        torch.set_num_threads(previous)
    return {
        "value": round(layer_bytes / per_layer / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "ops": "the reference's pytorch backend (nanovllm/layers/paged_kv/pytorch_backend.py:26-50) "
               "ported line for line: its validators, then its own torch ops (index_copy_ store, "
               "index_select gather) on host tensors; a port of the reference's Python code, which "
               "is read here, not imported",
        "sample": (f"decode step: {layers} of the 28 layers (store of the 256 new rows, then 256 x 2 "
                   f"per-sequence gathers of K and V) on host tensors, one layer-sized cache; "
                   f"median of {len(run_s)} runs ({layers * sum(run_s):.1f} s of CPU work), "
                   f"{per_layer:.3f} s per layer (runs {min(run_s):.3f}-{max(run_s):.3f})"),
        "seconds_per_layer": round(per_layer, 4),
        "seconds_per_layer_runs": [round(x, 4) for x in run_s],
        "decode_tokens_per_s_equivalent": round(wl.num_seqs / (per_layer * wl.num_layers), 3),
        "torch_threads": threads,
        "cpu_model": cpu_model(),
        "configs": configs,
    }


def openmp_port_baseline(wl, layers: int, repeats: int) -> dict:
    """The oracle's C restatement (OpenMP) on the host cores: one decode
    step of ``layers`` layers (pack, then per layer store + K/V varlen
    gather) against ONE layer-sized host cache reused by every layer (the
    full cache does not fit host memory), bytes counted as on the GPU.  A
    second CPU figure beside the reference's own torch ops."""
    import numpy as np
    import torch

    from oracle import c_oracle

    threads = c_oracle.default_threads()
    kc = np.full((wl.num_blocks, wl.block_size, wl.num_kv_heads, wl.head_dim), 0x3F80, dtype=np.int16)
    vc = np.full_like(kc, 0x3F80)
    tables = wl.padded_block_tables()
    offsets, ids = wl.csr()
    total = int(wl.num_tokens.sum())
    k_out = np.empty((total, wl.num_kv_heads, wl.head_dim), dtype=np.int16)
    v_out = np.empty_like(k_out)
    keys = wl.key.view(torch.int16).numpy()
    values = wl.value.view(torch.int16).numpy()

    def cpu_step():
        packed = c_oracle.pack_decode(wl.num_tokens, offsets, ids, wl.block_size, tables.shape[1])
        for layer in range(layers):
            c_oracle.store(keys[layer % keys.shape[0]], values[layer % values.shape[0]], kc, vc,
                           packed["slot_mapping"], threads=threads)
            c_oracle.gather_varlen(kc, packed["block_tables"], packed["cu_seqlens_k"], threads=threads, out=k_out)
            c_oracle.gather_varlen(vc, packed["block_tables"], packed["cu_seqlens_k"], threads=threads, out=v_out)

    cpu_step()  # first touch of the outputs
    times = []
    for _ in range(max(1, repeats)):
        t0 = time.perf_counter()
        cpu_step()
        times.append(time.perf_counter() - t0)
    seconds = sorted(times)[len(times) // 2]
    step_bytes = wl.store_bytes(layers=layers) + wl.gather_bytes(layers=layers)
    return {
        "value": round(step_bytes / seconds / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle C restatement (OpenMP, {threads} threads): pack + {layers} layers of "
                   f"store + K/V varlen gather of the same decode step against one layer-sized "
                   f"host cache, median of {max(1, repeats)} runs, {seconds:.2f} s each"),
        "decode_tokens_per_s_equivalent": round(wl.num_seqs / (seconds * wl.num_layers / layers), 2),
    }


if __name__ == "__main__":
    sys.exit(main())
