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
    ("void nkv::(anonymous namespace)::attn_decode_partial_kernel<8, 2, false>(int)",
     "attn_decode_partial_kernel<8, 2, false>"),
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
    assert profiling.algorithmic_bytes_for("grouped_decode_2x8") == {
        "attn_decode_mfma_kernel": total * 2 * 128 * 2 * 2 + 2 * 256 * 16 * 128 * 2}
