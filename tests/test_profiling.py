"""CPU tests of the rocprofv3 harness (nanokv.profiling): the commands it
builds, kernel-name shortening, the kernel-trace and counter CSV parsers,
the copy calibration and the summary, on small CSVs in rocprofv3's column
layout written by the tests."""
from __future__ import annotations

import csv
import json

import pytest

from nanokv import profiling

TRACE_COLUMNS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id",
                 "Kernel_Name", "Correlation_Id", "Start_Timestamp", "End_Timestamp", "LDS_Block_Size",
                 "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Workgroup_Size_X",
                 "Workgroup_Size_Y", "Workgroup_Size_Z", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
COUNTER_COLUMNS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
                   "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
                   "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
                   "Counter_Value", "Start_Timestamp", "End_Timestamp"]
STORE = ("void nkv::(anonymous namespace)::store_rows_kernel<16>(unsigned char const*, unsigned char "
         "const*, unsigned char*, unsigned char*, int const*, int, long, long, long, int, int, long)")
GATHER = ("void nkv::(anonymous namespace)::gather_planned_kernel<16, false>(unsigned char const*, "
          "unsigned char const*, HIP_vector_type<int, 4u> const*, int, int, long, long, long, "
          "unsigned char*, unsigned char*)")
COPY = "__amd_rocclr_copyBuffer(void*, void*, unsigned long)"


def write_trace(path, dispatches):
    with open(path, "w", newline="") as handle:
        w = csv.DictWriter(handle, TRACE_COLUMNS)
        w.writeheader()
        for i, (name, start, end) in enumerate(dispatches, 1):
            row = dict.fromkeys(TRACE_COLUMNS, 0)
            row.update(Kind="KERNEL_DISPATCH", Agent_Id="Agent 1", Dispatch_Id=i, Kernel_Name=name,
                       Start_Timestamp=start, End_Timestamp=end, Workgroup_Size_X=128,
                       Workgroup_Size_Y=1, Workgroup_Size_Z=1, Grid_Size_X=4096, Grid_Size_Y=2,
                       Grid_Size_Z=1)
            w.writerow(row)


def write_counters(path, rows):
    with open(path, "w", newline="") as handle:
        w = csv.DictWriter(handle, COUNTER_COLUMNS)
        w.writeheader()
        for dispatch, name, counter, value in rows:
            row = dict.fromkeys(COUNTER_COLUMNS, 0)
            row.update(Dispatch_Id=dispatch, Agent_Id="Agent 1", Kernel_Name=name,
                       Counter_Name=counter, Counter_Value=value)
            w.writerow(row)


@pytest.mark.parametrize("raw,short", [
    (STORE, "store_rows_kernel<16>"),
    (GATHER, "gather_planned_kernel<16, false>"),
    (COPY, "__amd_rocclr_copyBuffer"),
    ("void nkv::(anonymous namespace)::attn_decode_range_kernel<false, true>(int)",
     "attn_decode_range_kernel<false, true>"),
    ("void at::native::reduce_kernel<512, 1, at::native::ReduceOp<long, at::native::func_wrapper_t"
     "<long, at::native::sum_functor<long, long, long>::operator()(at::TensorIterator&)::{lambda(long,"
     " long)#1}>, unsigned int, long, 4, 4> >(at::native::ReduceOp<long>)", None),
])
def test_short_names(raw, short):
    got = profiling.short_name(raw)
    if short is None:
        assert got.startswith("reduce_kernel<512, 1,") and "(" not in got.split(">")[-1]
    else:
        assert got == short


def test_commands_put_the_program_right_after_the_separator():
    trace = profiling.trace_command("chunked_prefill", "out/trace", replay=7)
    assert trace[:3] == ["rocprofv3", "--kernel-trace", "--stats"]
    sep = trace.index("--")
    assert trace[sep + 1:] == ["python3", "bench.py", "--case", "chunked_prefill", "--profile-replay", "7"]
    pmc = profiling.counter_command("decode_step", "WRITE_SIZE", "out/w")
    assert pmc[:4] == ["timeout", "-s", "KILL", "120"] and pmc[4:7] == ["rocprofv3", "--pmc", "WRITE_SIZE"]
    assert "--kernel-trace" not in pmc and "--sys-trace" not in pmc
    copy = profiling.counter_command(None, "FETCH_SIZE", "out/c")
    assert copy[-2:] == ["--copy-calibration-mib", str(profiling.COPY_CALIBRATION_MIB)]
    with pytest.raises(ValueError):
        profiling.counter_command("decode_step", "FETCH_SIZE,WRITE_SIZE", "out")
    with pytest.raises(ValueError):
        profiling.trace_command("no_such_case", "out")
    plan = profiling.collection_plan("narrow_rows", profiling.Path("o"))
    assert [label for label, _ in plan] == ["trace", "fetch", "write", "copy_fetch", "copy_write"]


def test_kernel_durations_median_and_warmup(tmp_path):
    path = tmp_path / "t_kernel_trace.csv"
    # store durations 100 (warmup), 10, 12, 11, 30 ns; gather 1000, 2000 ns
    write_trace(path, [(STORE, 0, 100), (GATHER, 200, 1200), (STORE, 1300, 1310), (STORE, 1400, 1412),
                       (GATHER, 1500, 3500), (STORE, 3600, 3611), (STORE, 3700, 3730)])
    dispatches = profiling.read_kernel_trace(path)
    assert [d.dispatch_id for d in dispatches] == list(range(1, 8))
    assert dispatches[0].grid == (4096, 2, 1)
    stats = profiling.kernel_durations(dispatches, skip_first=1)
    store = stats["store_rows_kernel<16>"]
    assert store["dispatches"] == 4
    assert store["median_us"] == pytest.approx(0.0115)
    assert store["mean_us"] == pytest.approx(0.01575)
    assert stats["gather_planned_kernel<16, false>"]["median_us"] == pytest.approx(2.0)


def test_counters_copy_factor_and_summary(tmp_path):
    out = tmp_path / "run"
    for sub in ("trace", "fetch", "write", "copy_fetch", "copy_write"):
        (out / sub).mkdir(parents=True)
    write_trace(out / "trace" / "t_kernel_trace.csv",
                [(GATHER, 0, 1_000_000), (GATHER, 0, 2_000_000), (GATHER, 0, 2_000_000),
                 (GATHER, 0, 2_000_000)])
    mib = profiling.COPY_CALIBRATION_MIB
    # the copy's FETCH_SIZE reads half its bytes, WRITE_SIZE all of them (KiB)
    write_counters(out / "copy_fetch" / "c_counter_collection.csv",
                   [(1, COPY, "FETCH_SIZE", mib * 512.0)])
    write_counters(out / "copy_write" / "c_counter_collection.csv",
                   [(1, COPY, "WRITE_SIZE", mib * 1024.0)])
    # the gather: two dispatches, each counter reported in two parts per dispatch
    write_counters(out / "fetch" / "p_counter_collection.csv",
                   [(1, GATHER, "FETCH_SIZE", 1000.0), (1, GATHER, "FETCH_SIZE", 1000.0),
                    (2, GATHER, "FETCH_SIZE", 3000.0), (2, GATHER, "FETCH_SIZE", 1000.0)])
    write_counters(out / "write" / "p_counter_collection.csv",
                   [(1, GATHER, "WRITE_SIZE", 4000.0), (2, GATHER, "WRITE_SIZE", 4000.0)])
    rows = profiling.read_counters(out / "fetch" / "p_counter_collection.csv")
    means = profiling.counter_means(rows, "FETCH_SIZE")
    assert means["gather_planned_kernel<16, false>"] == {"dispatches": 2, "mean": 3000.0, "min": 2000.0,
                                                         "max": 4000.0}
    copy_rows = profiling.read_counters(out / "copy_fetch" / "c_counter_collection.csv")
    assert profiling.copy_factor(copy_rows, "FETCH_SIZE") == pytest.approx(0.5)
    summary = profiling.summarize("prefix_gather", out, {"gather_planned_kernel": 16_000_000},
                                  commands={"trace": ["rocprofv3", "--kernel-trace"]})
    gather = summary["kernels"]["gather_planned_kernel<16, false>"]
    assert gather["dispatches"] == 3 and gather["median_us"] == pytest.approx(2000.0)
    assert gather["achieved_gbps_at_median"] == pytest.approx(8.0)
    # 3000 KiB read at factor 0.5 -> 6000 KiB; 4000 KiB written at factor 1
    assert gather["hbm_read_bytes"] == 6000 * 1024 and gather["hbm_write_bytes"] == 4000 * 1024
    assert gather["traffic_over_algorithmic"] == pytest.approx(10000 * 1024 / 16_000_000)
    text = profiling.render_markdown(summary)
    assert "`gather_planned_kernel<16, false>` | 3 | 2000.00" in text
    assert "rocprofv3 --kernel-trace" in text
    json.dumps(summary)


def test_algorithmic_bytes_follow_the_workloads():
    from nanokv import workloads

    c2 = profiling.algorithmic_bytes_for("chunked_prefill")
    wl = workloads.build("chunked_prefill")
    assert c2 == {"store_rows_kernel": wl.store_bytes(layers=1),
                  "gather_planned_kernel": wl.gather_bytes(layers=1),
                  "store_gather_kernel": wl.store_gather_bytes(layers=1)}
    # the fused launch skips reading the 8192 new rows back (K and V, 2 KiB each)
    assert c2["store_gather_kernel"] == c2["store_rows_kernel"] + c2["gather_planned_kernel"] - 8192 * 2 * 2048
    assert set(profiling.algorithmic_bytes_for("decode_store")) == {"store_rows_kernel"}
    assert set(profiling.algorithmic_bytes_for("prefix_gather")) == {"gather_planned_kernel"}


def test_prefill_flops_match_the_bench_workload():
    import sys

    sys.path.insert(0, str(profiling.Path(__file__).resolve().parents[1]))
    import bench

    q_lens, k_lens = bench.chunked_prefill_shape()
    pairs = sum(sum(lk - lq + j + 1 for j in range(lq)) for lq, lk in zip(q_lens, k_lens))
    assert profiling.algorithmic_flops_for("prefill_attention") == {"attn_prefill_kernel": 4 * 128 * 16 * pairs}
    # 2 kv heads x 128 dims of K and V per context row, plus q and out of 16 query heads
    from nanokv import workloads

    total = int(workloads.build("decode_step", num_layers=1).num_tokens.sum())
    nbytes = total * 2 * 128 * 2 * 2 + 2 * 256 * 16 * 128 * 2
    assert profiling.algorithmic_bytes_for("grouped_decode_2x8") == {
        "attn_decode_entry_kernel": nbytes, "attn_decode_range_kernel": nbytes}


FAKE_ROCPROF = '''#!{python}
"""Stand-in for rocprofv3 in these CPU tests: writes a kernel trace of
{n} gather dispatches into the -d directory, prints the replay's last line
(or sleeps, or prints nothing, as the test asks)."""
import csv, os, sys, time
args = sys.argv[1:]
mode = os.environ.get("FAKE_ROCPROF_MODE", "ok")
if mode == "hang":
    time.sleep(60)
out = os.path.join(args[args.index("-d") + 1], "host")
os.makedirs(out, exist_ok=True)
columns = {columns!r}
with open(os.path.join(out, args[args.index("-o") + 1] + "_kernel_trace.csv"), "w", newline="") as f:
    w = csv.DictWriter(f, columns)
    w.writeheader()
    for i in range({n}):
        row = dict.fromkeys(columns, 0)
        row.update(Dispatch_Id=i + 1, Kernel_Name={gather!r}, Start_Timestamp=1000 * i,
                   End_Timestamp=1000 * i + (5000 if i == 0 else 1100 + i % 3 * 10))
        w.writerow(row)
if mode == "ok":
    print("profile replay complete: " + args[args.index("--case") + 1])
sys.exit(139 if mode == "ok" else 1)
'''


def fake_rocprof(tmp_path, monkeypatch, mode="ok", n=7):
    import sys

    bin_dir = tmp_path / "bin"
    bin_dir.mkdir()
    script = bin_dir / "rocprofv3"
    script.write_text(FAKE_ROCPROF.format(python=sys.executable, n=n, columns=TRACE_COLUMNS,
                                          gather=GATHER))
    script.chmod(0o755)
    monkeypatch.setenv("PATH", f"{bin_dir}:{__import__('os').environ['PATH']}")
    monkeypatch.setenv("FAKE_ROCPROF_MODE", mode)


def test_trace_on_this_host_reads_the_replays_kernel(tmp_path, monkeypatch):
    """trace_kernel_here runs the case's trace command as a child, skips the
    first dispatch, and keeps the trace even when the profiler exits
    non-zero after the replay's last line (as rocprofv3 can)."""
    fake_rocprof(tmp_path, monkeypatch, n=7)
    got = profiling.trace_kernel_here("decode_step", "gather_planned_kernel", replay=10, timeout_s=60)
    assert got["kernel"] == "gather_planned_kernel<16, false>"
    assert got["dispatches"] == 6  # the 5 us first dispatch skipped
    assert got["median_us"] == pytest.approx(1.11)
    assert got["mean_us"] == pytest.approx((1.11 + 1.12 + 1.10 + 1.11 + 1.12 + 1.10) / 6)
    assert got["rocprof_exit"] == 139
    command = got["command"].split()
    assert command[0] == "rocprofv3" and command[command.index("--") + 2].endswith("bench.py")
    assert command[-4:] == ["--case", "decode_step", "--profile-replay", "10"]


@pytest.mark.parametrize("mode,timeout,what", [("hang", 2, "did not finish"),
                                                ("silent", 60, "did not complete")])
def test_trace_on_this_host_reports_failures(tmp_path, monkeypatch, mode, timeout, what):
    fake_rocprof(tmp_path, monkeypatch, mode=mode)
    got = profiling.trace_kernel_here("decode_step", "gather_planned_kernel", timeout_s=timeout)
    assert what in got["error"]


def test_same_host_roofline_record():
    import bench

    trace = {"kernel": "gather_planned_kernel<16, false>", "dispatches": 270, "mean_us": 1150.0,
             "median_us": 1140.0, "command": "rocprofv3 ..."}
    got = bench.same_host_roofline(trace, 7_300_773_108, 1160.0)
    assert got["frac_at_mean"] == pytest.approx(7_300_773_108 / 1150e3 / 8000, abs=1e-4)
    assert got["events_over_trace_mean"] == pytest.approx(1160 / 1150, abs=1e-4)
    assert bench.same_host_roofline({"error": "x"}, 1, 1.0) == {"error": "x"}
    assert bench.same_host_roofline(None, 1, 1.0) is None


def test_trace_on_this_host_echoes_the_child(tmp_path, monkeypatch, capsys):
    """With echo the child's lines reach stderr as they arrive, so a slow
    child (a cold first import) is visible while the bench waits for it."""
    fake_rocprof(tmp_path, monkeypatch, n=3)
    got = profiling.trace_kernel_here("decode_step", "gather_planned_kernel", replay=10,
                                      timeout_s=60, echo=True)
    assert "error" not in got
    assert "[trace] profile replay complete: decode_step" in capsys.readouterr().err


def test_store_floor_phases_split_one_kernel_by_dispatch_order(tmp_path):
    """The store-floor replay launches the copy, then the store into
    contiguous slots, then into the workload's slots: the store's dispatches
    are labelled by order (first half, second half), trace and counters
    alike, and the copy is reported beside them with its own bytes."""
    out = tmp_path / "store_floor"
    for d in ("trace", "fetch", "write", "copy_fetch", "copy_write"):
        (out / d).mkdir(parents=True)
    dispatches = [(COPY, 0, 12_000)] * 3 + [(STORE, 0, 12_100)] * 3 + [(STORE, 0, 13_700)] * 3
    write_trace(out / "trace" / "t_kernel_trace.csv", dispatches)
    # a setup copy of another size before the replay: dropped (not the copy's modal grid)
    with open(out / "trace" / "t_kernel_trace.csv", newline="") as handle:
        rows = list(csv.DictReader(handle))
    setup = dict(rows[0], Dispatch_Id=0, End_Timestamp=900_000, Grid_Size_X=999_424)
    with open(out / "trace" / "t_kernel_trace.csv", "w", newline="") as handle:
        w = csv.DictWriter(handle, TRACE_COLUMNS)
        w.writeheader()
        w.writerows([setup] + rows)
    mib = 1024 * 1024
    write_counters(out / "copy_fetch" / "c_counter_collection.csv", [(1, COPY, "FETCH_SIZE", 512 * 1024)])
    write_counters(out / "copy_write" / "c_counter_collection.csv", [(1, COPY, "WRITE_SIZE", 1024 * 1024)])
    fetch = [(i, COPY, "FETCH_SIZE", 16 * 1024) for i in (1, 2, 3)]
    fetch += [(i, STORE, "FETCH_SIZE", 16 * 1024) for i in (4, 5, 6)]
    fetch += [(i, STORE, "FETCH_SIZE", 17 * 1024) for i in (7, 8, 9)]
    write_counters(out / "fetch" / "f_counter_collection.csv", fetch)
    write = [(i, COPY if i < 4 else STORE, "WRITE_SIZE", 32 * 1024) for i in range(1, 10)]
    write_counters(out / "write" / "w_counter_collection.csv", write)
    summary = profiling.summarize("store_floor", out, profiling.algorithmic_bytes_for("store_floor"))
    k = summary["kernels"]
    contiguous, scattered = ("store_rows_kernel<16> [contiguous slots]",
                             "store_rows_kernel<16> [chunked-prefill slots]")
    assert set(k) == {"__amd_rocclr_copyBuffer", contiguous, scattered}
    assert k[contiguous]["dispatches"] == 2 and k[contiguous]["median_us"] == pytest.approx(12.1)
    assert k[scattered]["median_us"] == pytest.approx(13.7)
    assert k["__amd_rocclr_copyBuffer"]["algorithmic_bytes"] == 67_108_864
    assert k["__amd_rocclr_copyBuffer"]["dispatches"] == 2          # 3 replayed, first skipped
    assert k["__amd_rocclr_copyBuffer"]["max_us"] == pytest.approx(12.0)
    assert k[contiguous]["hbm_read_bytes"] == 32 * mib and k[scattered]["hbm_read_bytes"] == 34 * mib
    assert k[scattered]["hbm_gbps_at_median"] == pytest.approx(66 * mib / 13_700)
    text = profiling.render_markdown(summary)
    assert "[contiguous slots]" in text and "HBM GB/s at median" in text
