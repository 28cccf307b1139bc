"""The bench's profile summarizers (CPU only): the kernel-trace grouping that the committed
trace summaries under profiles/ come from."""
from __future__ import annotations

import csv
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _trace(tmp_path, dispatches):
    """A rocprofv3-style kernel-trace CSV: (name, duration_ns, gap_before_ns) per dispatch."""
    rows, t = [], 0
    for name, dur, gap in dispatches:
        t += gap
        rows.append({"Kernel_Name": name, "Grid_Size_X": str(256 * 256),
                     "Workgroup_Size_X": "256", "Start_Timestamp": str(t),
                     "End_Timestamp": str(t + dur)})
        t += dur + 1000
    with open(os.path.join(tmp_path, "run_kernel_trace.csv"), "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=list(rows[0]))
        w.writeheader()
        w.writerows(rows)
    return str(tmp_path)


def _rows(text):
    out = []
    for line in text.splitlines()[3:]:
        parts = line.split()
        out.append((int(parts[0]), float(parts[1]), parts[-1]))
    return out


def test_runs_split_on_key_gap_and_duration(tmp_path):
    d = _trace(tmp_path,
               [("k_A", 50_000, 0)] * 5 +                 # shape 1
               [("k_A", 90_000, 5_000_000)] +             # shape 2 after a host pause
               [("k_A", 90_000, 0)] * 4 +
               [("k_A", 300_000, 0)] * 3 +                # shape 3, no pause: duration
               [("k_B", 40_000, 0)] * 2)
    rows = _rows(bench.summarize_trace_by_grid(d, "k_", "CMD", runs=True))
    assert rows == [(5, 50.0, "k_A"), (5, 90.0, "k_A"), (3, 300.0, "k_A"), (2, 40.0, "k_B")]


def test_runs_keep_strictly_alternating_keys_apart(tmp_path):
    # a long run of k_T, then two launches per call alternating k_F / k_T at other durations
    d = _trace(tmp_path, [("k_T", 1_570_000, 0)] * 3 +
               [("k_F", 357_000, 0), ("k_T", 380_000, 0)] * 4)
    rows = _rows(bench.summarize_trace_by_grid(d, "k_", "CMD", runs=True))
    assert rows == [(3, 1570.0, "k_T"), (4, 357.0, "k_F"), (4, 380.0, "k_T")]


def test_one_outlier_does_not_split_a_run(tmp_path):
    d = _trace(tmp_path, [("k_A", 100_000, 0)] * 3 + [("k_A", 200_000, 0)] +
               [("k_A", 100_000, 0)] * 3)
    rows = _rows(bench.summarize_trace_by_grid(d, "k_", "CMD", runs=True))
    assert rows[0][0] == 6 and rows[0][1] == 100.0
    assert (1, 200.0, "k_A") in rows


def test_without_runs_groups_by_key(tmp_path):
    d = _trace(tmp_path, [("k_A", 50_000, 0), ("k_B", 60_000, 0), ("k_A", 70_000, 0)])
    rows = _rows(bench.summarize_trace_by_grid(d, "k_", "CMD", runs=False))
    assert rows == [(2, 60.0, "k_A"), (1, 60.0, "k_B")]
