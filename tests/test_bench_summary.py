"""The benchmark's counter summaries: traffic from TCC-to-memory request counts
by size, calibrated by the runtime's 256 MiB copy, and the VALU table; and
that the benchmark line reads those tables back (no GPU needed)."""
import contextlib
import csv
import io
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402

FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size", "Kernel_Id",
          "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count",
          "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def write_pass(directory, dispatches):
    """dispatches: [(kernel name, grid, {counter: value})] as rocprofv3 writes them."""
    os.makedirs(directory, exist_ok=True)
    with open(os.path.join(directory, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f, quoting=csv.QUOTE_NONNUMERIC)
        w.writerow(FIELDS)
        for i, (name, grid, counters) in enumerate(dispatches, 1):
            for counter, value in counters.items():
                w.writerow([i, i, "Agent 1", 1, 1, 1, grid, i, name, 256, 0, 0, 32, 0, 32, counter, float(value), 0, 1])


def run_summary(*args):
    out = io.StringIO()
    with contextlib.redirect_stdout(out):
        bench.pmc_summary(*args)
    return out.getvalue()


def test_traffic_table_counts_request_sizes_and_applies_the_copy_calibration(tmp_path):
    copy = bench.COPY_BYTES
    silu = "void (anonymous namespace)::silu16(int)"
    fill = ("__amd_rocclr_copyBuffer", 131072, {"TCC_EA0_RDREQ_32B_sum": 0, "TCC_EA0_RDREQ_64B_sum": 7,
                                                 "TCC_EA0_RDREQ_128B_sum": 262144})  # set-up copies: ignored
    rd = [fill, fill,
          (silu, 999, {"TCC_EA0_RDREQ_32B_sum": 10, "TCC_EA0_RDREQ_64B_sum": 20, "TCC_EA0_RDREQ_128B_sum": 30}),
          (silu, 999, {"TCC_EA0_RDREQ_32B_sum": 30, "TCC_EA0_RDREQ_64B_sum": 20, "TCC_EA0_RDREQ_128B_sum": 10}),
          # the calibration copies run last and read 2% more than they should:
          # every case is scaled by 1/1.02
          ("__amd_rocclr_copyBuffer", 131072, {"TCC_EA0_RDREQ_32B_sum": 0, "TCC_EA0_RDREQ_64B_sum": 0,
                                                "TCC_EA0_RDREQ_128B_sum": 1.02 * copy / 128})]
    rd.append(rd[-1])
    wr = [(silu, 999, {"TCC_EA0_WRREQ_sum": 100, "TCC_EA0_WRREQ_64B_sum": 40}),
          ("__amd_rocclr_copyBuffer", 131072, {"TCC_EA0_WRREQ_sum": copy / 64, "TCC_EA0_WRREQ_64B_sum": copy / 64})]
    write_pass(tmp_path / "rd", rd)
    write_pass(tmp_path / "wr", wr)
    alg = {case: 1000 for case in bench.TRAFFIC_CASES}
    text = run_summary("traffic", [str(tmp_path / "rd"), str(tmp_path / "wr")], alg)
    assert "read factor 0.9804" in text and "write factor 1.0000" in text
    # silu: mean read = (32*20 + 64*20 + 128*20) = 4480 B, /1.02; write = 32*60 + 64*40 = 4480 B.
    want_read, want_write = 4480 / 1.02, 4480
    (tmp_path / "summary.txt").write_text(text)
    rows = bench.summary_rows(str(tmp_path / "summary.txt"), 7)
    assert set(rows) == {bench.COPY_CASE, "silu_8192x6144"}
    silu = rows["silu_8192x6144"]
    assert silu[1] == "silu16"
    assert abs(float(silu[2]) - want_read) <= 0.5 and abs(float(silu[3]) - want_write) <= 0.5
    assert int(silu[4]) == round(want_read + want_write)
    assert abs(float(silu[6]) - (want_read + want_write) / 1000) < 1e-3
    assert int(rows[bench.COPY_CASE][4]) == 2 * copy  # the copy reads itself back exactly


def test_valu_table_splits_the_sampling_cases_in_launch_order(tmp_path):
    name = "void (anonymous namespace)::sample_paired<20>(...)"
    ds = []
    for valu in (100, 200, 300):  # mixed, greedy, Gumbel: two dispatches each
        for _ in range(2):
            ds.append((name, 1 << 18, {"SQ_INSTS_VALU": valu * 1e6, "SQ_WAVES": 4096, "SQ_INSTS_SALU": 1,
                                       "SQ_INSTS_LDS": 2, "SQ_INSTS_VMEM": 3}))
    write_pass(tmp_path / "sq", ds)
    text = run_summary("valu", [str(tmp_path / "sq")], {})
    (tmp_path / "valu.txt").write_text(text)
    rows = bench.summary_rows(str(tmp_path / "valu.txt"), 9)
    assert {k: int(v[1]) for k, v in rows.items()} == {"sampling_256x151936": 100_000_000,
                                                       "sampling_greedy": 200_000_000,
                                                       "sampling_gumbel": 300_000_000}
    assert rows["sampling_gumbel"][-1] == "2"


def test_committed_summaries_feed_the_benchmark_line():
    traffic = {case: bench.measured_traffic(case) for case in bench.TRAFFIC_CASES}
    alg = bench.traffic_case_bytes()
    for case, b in traffic.items():
        if b is None:
            pytest.fail(f"{bench.TRAFFIC_SUMMARY} has no row for {case}")
        assert 0.9 < b / alg[case] < 1.2, (case, b, alg[case])
    for case in ("sampling_256x151936", "sampling_greedy", "sampling_gumbel"):
        assert bench.measured_valu(case) is not None, case


def test_kernel_trace_dispatches_are_assigned_to_cases_in_order():
    """The child runs each case as (warm + rounds) x launches dispatches of one
    kernel; the timed part's median is the case's kernel time."""
    order = [{"case": "a", "launches": 2, "warm": 1, "rounds": 3}, {"case": "b", "launches": 1, "warm": 2, "rounds": 3}]
    disp = []
    t = 0
    for dur in [50.0, 50.0] + [10.0, 11.0, 12.0, 13.0, 14.0, 15.0]:  # case a: 2 warm dispatches, 6 timed
        disp.append((t, dur, "void (anonymous namespace)::ka<1>(int)"))
        t += 100
    for dur in [90.0, 90.0, 7.0, 5.0, 6.0]:  # case b: 2 warm, 3 timed
        disp.append((t, dur, "void kb(float)"))
        t += 100
    res, status = bench.assign_dispatches(order, disp[::-1])  # any input order: sorted by start
    assert status == "ok"
    assert res["a"] == ("ka<1>", 12.5, 6)
    assert res["b"] == ("kb", 6.0, 3)


@pytest.mark.parametrize("drop,extra", [(1, 0), (0, 1)])
def test_kernel_trace_that_does_not_line_up_is_refused(drop, extra):
    order = [{"case": "a", "launches": 1, "warm": 1, "rounds": 2}, {"case": "b", "launches": 1, "warm": 1, "rounds": 2}]
    disp = [(i, 1.0, "ka") for i in range(3)] + [(10 + i, 1.0, "kb") for i in range(3)]
    disp = disp[drop:] + [(100 + i, 1.0, "kb") for i in range(extra)]
    res, status = bench.assign_dispatches(order, disp)
    assert res == {} and status != "ok"


def test_slot_layouts_fold_into_their_case_with_min_and_median():
    kernels = {"kv": {"us": 20.0, "frac": 0.70, "kernel_us": 19.0, "kernel_frac": 0.74},
               "kv@identity": {"us": 22.0, "frac": 0.64, "kernel_us": 21.0, "kernel_frac": 0.67},
               "kv@perm1": {"us": 21.0, "frac": 0.67, "kernel_us": 20.0, "kernel_frac": 0.70},
               "other": {"us": 1.0, "frac": 0.1}}
    bench.fold_layouts(kernels)
    assert set(kernels) == {"kv", "other"}
    sweep = kernels["kv"]["layout_sweep"]
    assert sweep["layouts"] == 3
    assert sweep["frac_min"] == 0.64 and sweep["frac_median"] == 0.67
    assert sweep["kernel_frac_min"] == 0.67 and sweep["kernel_frac_median"] == 0.70
    assert kernels["kv"]["layouts"]["identity"]["kernel_us"] == 21.0


def test_copy_ceiling_compares_with_the_copy_of_about_the_same_traffic():
    kernels = {"copy_64mb": {"bytes": 64_000_000, "us": 12.0, "kernel_us": 10.0},
               "copy_128mb": {"bytes": 128_000_000, "us": 22.0},
               "add_rms_8192x1024": {"bytes": 67_000_000, "us": 12.0, "kernel_us": 11.0},
               "silu_8192x6144": {"bytes": 151_000_000, "us": 26.0, "kernel_us": 24.0},
               "rms_8x1024": {"bytes": 34_816, "us": 2.0}}
    bench.add_copy_ceilings(kernels)
    c = kernels["add_rms_8192x1024"]["copy_ceiling"]
    # kernel time on both sides: 67 MB / 11 us against 64 MB / 10 us
    assert c["case"] == "copy_64mb" and c["time"] == "kernel_us"
    assert c["GB/s"] == 6400.0 and c["frac"] == round((67e6 / 11.0) / (64e6 / 10.0), 4)
    # the 128 MiB copy has no kernel time: both sides by event time
    c = kernels["silu_8192x6144"]["copy_ceiling"]
    assert c["case"] == "copy_128mb" and c["time"] == "us"
    assert c["frac"] == round((151e6 / 26.0) / (128e6 / 22.0), 4)
    assert "copy_ceiling" not in kernels["rms_8x1024"] and "copy_ceiling" not in kernels["copy_64mb"]
    # no copy case measured: no field
    alone = {"qkv_rope_8192": {"bytes": 136_000_000, "us": 25.0}}
    bench.add_copy_ceilings(alone)
    assert "copy_ceiling" not in alone["qkv_rope_8192"]


def test_sweep_slot_layouts_are_distinct_slots_inside_the_cache():
    for tokens, blocks in ((8192, 32), (16384, 128)):
        layouts = bench.slot_layouts(tokens, blocks)
        assert [t for t, _ in layouts] == ["@identity"] + [f"@perm{s}" for s in bench.LAYOUT_SEEDS]
        for _, slots in layouts:
            assert len(np.unique(slots)) == tokens
            assert slots.min() >= 0 and slots.max() < blocks * bench.BS
            # whole 256-token blocks stay together (slot % 256 == token % 256)
            assert np.array_equal(slots % bench.BS, np.arange(tokens) % bench.BS)


def test_kernel_trace_child_is_not_started_under_a_profiler():
    assert bench.under_profiler({"LD_PRELOAD": "/opt/rocm/lib/librocprofiler-sdk-tool.so"})
    assert bench.under_profiler({"ROCPROF_COUNTERS": "pmc: SQ_WAVES"})
    assert not bench.under_profiler({"LD_PRELOAD": "", "PATH": "/usr/bin"})
