"""fast_kernels.benchmarking.rocprof on synthetic rocprofv3 CSV: dispatches grouped by (kernel,
grid), and the duration split that separates two shapes sharing one kernel and grid."""

from __future__ import annotations

import csv
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parent.parent / "fast-kernels_amd"))

from fast_kernels.benchmarking.rocprof import kernel_trace_by_grid  # noqa: E402

FIELDS = ["Kind", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Workgroup_Size_X",
          "Grid_Size_X", "Grid_Size_Y"]
KERNEL = "void fk::w4a16_gemv_stream_kernel<128, 2>(fk::GemvParams)"


def _write(d: Path, rows: list[tuple[str, int, int]]) -> Path:
    d.mkdir(parents=True)
    with (d / "x_kernel_trace.csv").open("w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=FIELDS)
        w.writeheader()
        t = 0
        for name, grid, dur_ns in rows:
            w.writerow({"Kind": "KERNEL_DISPATCH", "Kernel_Name": name, "Start_Timestamp": t,
                        "End_Timestamp": t + dur_ns, "Workgroup_Size_X": 512,
                        "Grid_Size_X": grid, "Grid_Size_Y": 1})
            t += dur_ns + 1000
    return d


def test_grouping_and_split(tmp_path: Path) -> None:
    rows = [(KERNEL, 131072, 7000)] * 30 + [(KERNEL, 131072, 38000)] * 30
    rows += [(KERNEL, 147456, 9800)] * 10 + [("void other(int)", 64, 100)]
    d = _write(tmp_path / "a", rows)
    plain = kernel_trace_by_grid(d, "w4a16")
    assert len(plain) == 2
    both = next(r for r in plain if r["grid_threads"] == 131072)
    assert both["calls"] == 60 and abs(both["avg_us"] - 22.5) < 1e-9
    assert both["workgroups"] == 256
    split = kernel_trace_by_grid(d, "w4a16", split_us=20)
    rows_131 = sorted((r for r in split if r["grid_threads"] == 131072), key=lambda r: r["avg_us"])
    assert [r["calls"] for r in rows_131] == [30, 30]
    assert abs(rows_131[0]["avg_us"] - 7.0) < 1e-9 and abs(rows_131[1]["avg_us"] - 38.0) < 1e-9
    assert rows_131[0]["kernel"].endswith("[< 20 us]")
    assert rows_131[1]["kernel"].endswith("[>= 20 us]")


def test_split_keeps_outliers_in_their_row(tmp_path: Path) -> None:
    d = _write(tmp_path / "b", [(KERNEL, 131072, 7000)] * 50 + [(KERNEL, 131072, 25000)] * 2)
    rows = kernel_trace_by_grid(d, "w4a16", split_us=20)
    assert len(rows) == 1 and rows[0]["calls"] == 52


def test_split_keeps_one_shape_across_the_cut(tmp_path: Path) -> None:
    # one shape whose durations straddle the cut (medians 19.9 and 20.4 us) stays one row
    d = _write(tmp_path / "c", [(KERNEL, 131072, 19900)] * 25 + [(KERNEL, 131072, 20400)] * 75)
    rows = kernel_trace_by_grid(d, "w4a16", split_us=20)
    assert len(rows) == 1 and rows[0]["calls"] == 100
