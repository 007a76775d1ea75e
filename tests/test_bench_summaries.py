"""The measurement script's own arithmetic, on the CPU: the busy time of
overlapping launches, the runs it finds in a kernel trace (each from its
pack_rows_kernel to its pooling), and the timed-run paragraph it writes
from a synthetic trace and bench line. No GPU and no profiler: the inputs
are made here with known answers."""
import csv
import json

import pytest

import bench


def test_busy_union_counts_overlap_once():
    iv = [("gemm_qkv", 0.0, 2.0), ("gemm_out", 1.0, 3.0), ("attention", 2.5, 9.0), ("gemm_ffn_in", 5.0, 6.0)]
    assert bench.busy_union(iv, {"gemm_qkv", "gemm_out", "gemm_ffn_in"}) == pytest.approx(4.0)
    assert bench.busy_union(iv, {"attention"}) == pytest.approx(6.5)
    # One interval inside another adds nothing; touching ones add up.
    assert bench.busy_union([("a", 0, 10), ("a", 2, 3), ("a", 10, 12)], {"a"}) == pytest.approx(12.0)
    assert bench.busy_union(iv, {"nothing"}) == 0.0


def test_run_slice_takes_a_run_from_its_packing_to_its_pooling():
    names = ["copy", "pack_rows_kernel", "gemm_a", "pool_kernel", "probe",
             "pack_rows_kernel", "gemm_b", "gemm_c", "pool_part_kernel", "pool_kernel", "mfma_probe_kernel",
             "pack_rows_kernel", "gemm_d"]
    same = lambda x: x  # noqa: E731
    assert bench.run_slice(names, 0, same) == ["pack_rows_kernel", "gemm_a", "pool_kernel"]
    assert bench.run_slice(names, 1, same) == ["pack_rows_kernel", "gemm_b", "gemm_c", "pool_part_kernel",
                                               "pool_kernel"]
    # A run cut short (no pooling yet) runs to the end of what was traced.
    assert bench.run_slice(names, 2, same) == ["pack_rows_kernel", "gemm_d"]
    assert bench.run_slice(names, 3, same) is None


def _trace(tmp_path, rows):
    d = tmp_path / "prof"
    d.mkdir()
    with open(d / "run_kernel_trace.csv", "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Stream_Id"])
        w.writeheader()
        for name, a, b, st in rows:
            w.writerow({"Kernel_Name": name, "Start_Timestamp": a, "End_Timestamp": b, "Stream_Id": st})
    return d


def test_timed_run_paragraph_reads_the_named_runs(tmp_path):
    # Run 0: a split run, two overlapping GEMM launches on streams 1 and 2
    # (busy 3000 ns of 4000 summed). Run 1: the whole-batch run, two GEMM
    # launches one after the other, then the bench's probe far later, which
    # must not stretch the run.
    us = 1000   # (timestamps in ns)
    d = _trace(tmp_path, [
        ("pack_rows_kernel", 0, 100 * us, 1), ("gemm_lds_kernel<a>", 1000 * us, 3000 * us, 1),
        ("gemm_lds_kernel<a>", 2000 * us, 4000 * us, 2), ("pool_kernel", 4100 * us, 4200 * us, 1),
        ("pack_rows_kernel", 10000 * us, 10100 * us, 1), ("gemm_lds_kernel<b>", 10200 * us, 11200 * us, 1),
        ("gemm_lds_kernel<b>", 11300 * us, 13300 * us, 1), ("pool_kernel", 13400 * us, 14000 * us, 1),
        ("mfma_probe_kernel", 900000 * us, 990000 * us, 1),
    ])
    line = {"metric": "m", "roofline": {
        "timed_run_index": 1, "launches_per_step": 2, "avg_launch_us": 1.6, "launch_ms_per_step": 0.0032,
        "timed_run_ms": 0.0041, "achieved": 900.0, "unit": "TFLOP/s", "frac": 0.36,
        "concurrent": {"timed_run_index": 0, "launches_per_step": 2, "avg_launch_us": 2.1, "busy_us_per_step": 3.1,
                       "achieved": 800.0}}}
    log = tmp_path / "bench.log"
    log.write_text("# noise\n" + json.dumps(line) + "\n")
    text = "\n".join(bench.timed_run_from_trace(str(d), str(log)))
    # Whole batch: (1000 + 2000) / 2 us a launch, 3 ms of launches in the
    # run's 4 ms (from its packing to its pooling, the probe left out).
    assert "run 1 of the command, stream(s) 1)" in text
    assert "2 GEMM launches, average 1500.0 µs a launch, 3.00 ms in all within the run's 4.00 ms" in text
    # Split: 2000 us a launch, busy 3000 us (the union), streams 1 and 2.
    assert "run 0, its parts side by side when it splits; stream(s) 1, 2)" in text
    assert "average 2000.0 µs a launch (overlapping), busy 3000 µs" in text
