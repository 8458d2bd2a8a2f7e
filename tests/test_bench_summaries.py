"""CPU tests of bench.py's rocprof summaries (the code that writes profiles/):
counter medians, shader clock and MFMA-pipe utilisation, and the HBM traffic
table scaled by a copy kernel of known bytes."""
from __future__ import annotations

import csv
import os

import pytest

import bench

HEADER = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id",
          "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size",
          "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count", "SGPR_Count", "Counter_Name",
          "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def write_counters(path, dispatches):
    """dispatches: (kernel name, duration ns, {counter: value}) in launch order."""
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(HEADER)
        t = 1_000_000
        for i, (name, ns, counters) in enumerate(dispatches, start=1):
            for c, v in counters.items():
                w.writerow([i, i, "Agent 1", 1, 7, 7, 65536, 3, name, 256, 0, 0, 128, 0, 64, c, v,
                            t, t + ns])
            t += ns + 1000


def test_counter_summary_clock_and_mfma_utilisation(tmp_path):
    d = tmp_path / "pmc"
    d.mkdir()
    # 8 XCDs x 1.5e6 cycles over 1 ms = 1.5 GHz; MFMA busy = 0.75 of 1.5e6 x 1024 SIMDs.
    busy = 0.75 * 1.5e6 * 1024
    rows = [("void k_gemm(int)", 1_000_000, {"GRBM_GUI_ACTIVE": 8 * 1.5e6,
                                               "SQ_VALU_MFMA_BUSY_CYCLES": busy})] * 3
    rows += [("void k_gemm(int)", 1_000_000, {"GRBM_GUI_ACTIVE": 8 * 1.5e6,
                                                "SQ_VALU_MFMA_BUSY_CYCLES": busy})] * 4
    write_counters(d / "run_counter_collection.csv", rows)
    text = bench.summarize_counters(str(d), skip=3, command="rocprofv3 ...")
    line = next(l for l in text.splitlines() if l.startswith("| `k_gemm`"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[1] == "4"  # the first 3 dispatches dropped
    assert cells[2] == "1000000"
    assert cells[-2] == "1.50 GHz"
    assert cells[-1] == "75%"
    assert "rocprofv3 ..." in text


def test_traffic_table_scales_by_the_copy_kernel(tmp_path):
    fetch, write = tmp_path / "f", tmp_path / "w"
    fetch.mkdir()
    write.mkdir()
    copy_bytes = 1 << 20
    # The counters read half the copy's bytes fetched and all its bytes written
    # (KiB per dispatch); a transpose-like kernel reads and writes the same.
    half = copy_bytes / 2 / 1024
    full = copy_bytes / 1024
    write_counters(fetch / "run_counter_collection.csv",
                   [("copy_k", 1000, {"FETCH_SIZE": half}), ("xpose_k", 1000, {"FETCH_SIZE": half}),
                    ("xpose_k", 1000, {"FETCH_SIZE": 3 * half})])
    write_counters(write / "run_counter_collection.csv",
                   [("copy_k", 1000, {"WRITE_SIZE": full}), ("xpose_k", 1000, {"WRITE_SIZE": full}),
                    ("xpose_k", 1000, {"WRITE_SIZE": full})])
    text = bench.summarize_traffic_table(str(fetch), str(write), skip=0, command="a ;; b",
                                         copy_kernel="copy_k", copy_bytes=copy_bytes)
    assert "FETCH_SIZE x 2.000, WRITE_SIZE x 1.000" in text
    line = next(l for l in text.splitlines() if l.startswith("| `xpose_k`"))
    cells = [c.strip() for c in line.strip("|").split("|")]
    # median of (1, 3) x half KiB = 2 x half -> 2 x copy bytes read
    assert float(cells[3]) == pytest.approx(2 * copy_bytes / 1e6, abs=0.01)
    assert float(cells[4]) == pytest.approx(copy_bytes / 1e6, abs=0.01)
    assert "    a" in text and "    b" in text
