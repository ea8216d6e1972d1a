"""profiles/ summaries: every case's dispatches are told apart in rocprofv3
CSVs of the one bench command (kernel symbol + grid size, then launch order
for c5 and c5x25, which share both), and counters become bytes through the
copy-kernel calibration.  Synthetic CSVs in the layout rocprofv3 writes."""

from __future__ import annotations

import csv
import json
import os

import pytest

from tilegen_amd import profiling as pf

_TRACE_COLS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id",
               "Kernel_Id", "Kernel_Name", "Correlation_Id", "Start_Timestamp",
               "End_Timestamp", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
               "Accum_VGPR_Count", "SGPR_Count", "Workgroup_Size_X", "Workgroup_Size_Y",
               "Workgroup_Size_Z", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
_PMC_COLS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id",
             "Thread_Id", "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size",
             "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count",
             "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def _dispatches(plan, dur_us, extra=True):
    """(start ns, name, grid, duration us) in the bench's launch order, with a
    stray unrelated kernel between the cases."""
    t, out = 1_000_000, []
    for case, sym, grid, n, _timed in plan:
        for i in range(n):
            out.append((t, sym, grid, dur_us[case] + 0.001 * (i % 3)))
            t += 50_000
        if extra:
            out.append((t, "rocsparse_other", grid, 1.0))
            t += 50_000
    return out


def _write_trace(d, rows):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "trace_kernel_trace.csv"), "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=_TRACE_COLS)
        w.writeheader()
        for k, (t, name, grid, us) in enumerate(rows):
            w.writerow({"Kind": "KERNEL_DISPATCH", "Dispatch_Id": k, "Kernel_Name": name,
                        "Start_Timestamp": t, "End_Timestamp": t + int(round(us * 1000)),
                        "Grid_Size_X": grid})


def _write_pmc(d, rows, counter, value_of):
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "pmc_counter_collection.csv"), "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=_PMC_COLS)
        w.writeheader()
        for k, (t, name, grid, _us) in enumerate(rows):
            w.writerow({"Dispatch_Id": k, "Kernel_Name": name, "Grid_Size": grid,
                        "Counter_Name": counter, "Counter_Value": value_of(name, grid, t),
                        "Start_Timestamp": t, "End_Timestamp": t + 1000})


@pytest.fixture(scope="module")
def plans():
    return (pf.case_plan(pf.STEPS, pf.WARMUP, pf.CASE_ITERS),
            pf.case_plan(pf.STEPS, pf.WARMUP, pf.PMC_CASE_ITERS))


def test_case_plan_counts_and_shared_grid(plans):
    plan, _ = plans
    by = {c: (sym, g, n, timed) for c, sym, g, n, timed in plan}
    assert [c for c, *_ in plan] == list(pf.CASE_ORDER)
    # headline: check + warmup + host-timed steps + warmup + event-timed steps
    assert by["c1"][2] == 1 + 2 * pf.WARMUP + 2 * pf.STEPS and by["c1"][3] == pf.STEPS
    # the others: check + one launch per input copy + warmup + event-timed launches
    from tilegen_amd.matrices import compulsory_bytes, make_baseline
    A = make_baseline("c2")
    copies = pf.bench_copies(compulsory_bytes("spmv", A.shape[0], A.shape[1], int(A.nnz), 1))
    assert copies == 25  # 27.2 MB a launch: 640 MiB of rotation
    assert by["c2"][2] == 1 + copies + pf.WARMUP + pf.CASE_ITERS
    assert pf.bench_copies(1 << 40) == 2 and pf.bench_copies(1) == 64
    assert by["c5"][:2] == by["c5x25"][:2]  # same kernel and grid: told apart by order
    spmv = [g for c, (s, g, _n, _t) in by.items() if s == "spmv_kernel"]
    assert len(set(spmv)) == len(spmv)


def test_summarize_splits_cases_and_scales_counters(plans, tmp_path):
    plan, pmc_plan = plans
    dur = {c: 10.0 * (i + 1) for i, c in enumerate(pf.CASE_ORDER)}
    root = str(tmp_path / "prof")
    _write_trace(os.path.join(root, "trace"), _dispatches(plan, dur))
    rows = _dispatches(pmc_plan, dur)
    kib = {c: 1000.0 * (i + 1) for i, c in enumerate(pf.CASE_ORDER)}
    order = {}
    for case, sym, grid, n, _ in pmc_plan:
        order.setdefault((sym, grid), []).append((case, n))

    def value(name, grid, t):
        # the k-th dispatch of (name, grid) belongs to the case that owns that slot
        seen = value.count.setdefault((name, grid), 0)
        value.count[(name, grid)] = seen + 1
        for case, n in order.get((name, grid), []):
            if seen < n:
                return kib[case]
            seen -= n
        return 7.0
    value.count = {}
    _write_pmc(os.path.join(root, "fetch"), rows, "FETCH_SIZE", value)
    value.count = {}
    _write_pmc(os.path.join(root, "write"), rows, "WRITE_SIZE", lambda *a: 64.0)
    copy = [(5, "tg_copy_kernel", 1 << 20, 1.0)] * 3
    mib = pf.COPY_MIB << 10  # KiB moved by the copy
    _write_pmc(os.path.join(root, "copy_fetch"), copy, "FETCH_SIZE", lambda *a: mib / 2)
    _write_pmc(os.path.join(root, "copy_write"), copy, "WRITE_SIZE", lambda *a: mib)
    bench = {"kernel_us_avg": 10.0, "cases": {c: {"us": dur[c]} for c in pf.CASE_ORDER[1:]}}
    bj = tmp_path / "bench.json"
    bj.write_text("[bench] noise\n" + json.dumps(bench) + "\n")
    out_dir = str(tmp_path / "profiles")
    s = pf.summarize(root, out_dir, str(bj))
    assert sorted(s) == sorted(pf.CASE_ORDER)
    for case, v in s.items():
        assert v["trace"]["calls"] == dict((c, n) for c, _s, _g, n, _t in plan)[case]
        assert abs(v["trace"]["avg_us"] - dur[case]) < 0.01, case
        assert v["fetch_size_kib"] == kib[case], case
        # FETCH_SIZE read half the copy's bytes: scaled by 2; WRITE_SIZE by 1
        assert v["beyond_l2_read_bytes_per_launch"] == pytest.approx(2 * kib[case] * 1024)
        assert v["beyond_l2_write_bytes_per_launch"] == pytest.approx(64.0 * 1024)
        assert os.path.exists(os.path.join(out_dir, "%s_%s.md" % (v["kernel"][:-7], case)))
    assert "| c5x25 |" in open(os.path.join(out_dir, "bench_cases.md")).read()


def test_missing_dispatches_are_reported(plans, tmp_path):
    plan, _ = plans
    rows = [r for r in _dispatches(plan, {c: 1.0 for c in pf.CASE_ORDER}) if r[1] != "spmm_kernel"]
    root = str(tmp_path)
    _write_trace(os.path.join(root, "trace"), rows)
    got = pf.trace_rows(os.path.join(root, "trace"), plan)
    assert got["c4"].size == 0 and got["c5"].size == dict(
        (c, n) for c, _s, _g, n, _t in plan)["c5"]
