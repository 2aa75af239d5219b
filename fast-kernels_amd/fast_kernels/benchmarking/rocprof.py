"""Summaries of rocprofv3 CSV output for the W4A16 kernels.

The benchmark runner's counter support: rocprofv3 writes one row per dispatch
(``*_kernel_trace.csv`` with --kernel-trace, ``*_counter_collection.csv`` with --pmc); the GEMV
kernel keeps one name for every shape, so dispatches are grouped by (kernel, grid size), which
identifies the shape. HBM traffic per launch comes from FETCH_SIZE and WRITE_SIZE (KiB per
dispatch), each scaled by what the same counter reports for a plain device-to-device copy of
known size (``bench.py --copy-calibration``): on gfx950 FETCH_SIZE counts 64 B per 128 B read
request, so the measured read scale is about 2.

Usage:
  python -m fast_kernels.benchmarking.rocprof trace DIR [--filter w4a16]
  python -m fast_kernels.benchmarking.rocprof traffic --fetch DIR --write DIR \\
      --copy-fetch DIR --copy-write DIR [--copy-bytes N] [--filter w4a16]
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import sys
from collections import defaultdict
from pathlib import Path

COPY_CALIBRATION_BYTES = 256 * 1024 * 1024


def short_kernel_name(name: str) -> str:
    """Kernel name without return type, namespaces and parameter list."""
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and i > 0 and name[i - 1] not in ":":
            name = name[:i]
            break
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    name = re.sub(r"\b\w+::", "", name)
    return name


def _find(directory: str | Path, suffix: str) -> Path:
    hits = sorted(Path(directory).rglob(f"*{suffix}"))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    return hits[0]


def kernel_trace_by_grid(directory: str | Path, name_filter: str = "",
                         split_us: float | None = None) -> list[dict]:
    """Per (kernel, grid) dispatch-duration statistics from a --kernel-trace CSV. split_us: a group
    whose dispatches fall on both sides of that duration, at least a tenth of them on each and the
    two sides' medians at least twice apart (two shapes with one kernel and grid, e.g. bench.py's
    70B o and gate_up, not one shape whose spread straddles the cut), is reported as two rows, the
    kernel name suffixed with the side."""
    path = _find(directory, "_kernel_trace.csv")
    groups: dict[tuple[str, int, int], list[int]] = defaultdict(list)
    with path.open(newline="") as fh:
        for row in csv.DictReader(fh):
            name = row["Kernel_Name"]
            if name_filter and name_filter not in name:
                continue
            grid = int(row["Grid_Size_X"]) * int(row.get("Grid_Size_Y", 1) or 1)
            wg = int(row["Workgroup_Size_X"])
            groups[(name, grid, wg)].append(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
    if split_us is not None:
        cut = int(split_us * 1e3)
        split: dict[tuple[str, int, int], list[int]] = {}
        for (name, grid, wg), durs in groups.items():
            lo = [d for d in durs if d < cut]
            hi = [d for d in durs if d >= cut]
            two = min(len(lo), len(hi)) >= 0.1 * len(durs)  # two populations, not outliers
            if two and sorted(hi)[len(hi) // 2] >= 2 * sorted(lo)[len(lo) // 2]:
                split[(f"{name} [< {split_us:g} us]", grid, wg)] = lo
                split[(f"{name} [>= {split_us:g} us]", grid, wg)] = hi
            else:
                split[(name, grid, wg)] = durs
        groups = split
    out = []
    for (name, grid, wg), durs in groups.items():
        durs.sort()
        label = short_kernel_name(name)
        if name.endswith(" us]"):
            label += " " + name[name.rindex("["):]
        out.append(
            {
                "kernel": label,
                "grid_threads": grid,
                "workgroups": grid // max(wg, 1),
                "calls": len(durs),
                "avg_us": sum(durs) / len(durs) / 1e3,
                "median_us": durs[len(durs) // 2] / 1e3,
                "min_us": durs[0] / 1e3,
                "max_us": durs[-1] / 1e3,
            }
        )
    out.sort(key=lambda r: -r["avg_us"] * r["calls"])
    return out


def counter_by_grid(directory: str | Path, counter: str, name_filter: str = "",
                    with_counts: bool = False) -> dict:
    """Mean counter value per (kernel, grid) from a --pmc counter-collection CSV (with_counts:
    (mean, dispatches) per key)."""
    path = _find(directory, "_counter_collection.csv")
    groups: dict[tuple[str, int], list[float]] = defaultdict(list)
    with path.open(newline="") as fh:
        for row in csv.DictReader(fh):
            if row["Counter_Name"] != counter:
                continue
            name = row["Kernel_Name"]
            if name_filter and name_filter not in name:
                continue
            groups[(short_kernel_name(name), int(row["Grid_Size"]))].append(float(row["Counter_Value"]))
    if with_counts:
        return {k: (sum(v) / len(v), len(v)) for k, v in groups.items()}
    return {k: sum(v) / len(v) for k, v in groups.items()}


def copy_scale(directory: str | Path, counter: str, copy_bytes: int) -> float:
    """Bytes per counter KiB, from the copy-calibration run (largest copy dispatch)."""
    values = counter_by_grid(directory, counter, "copy")
    if not values:
        values = counter_by_grid(directory, counter)
    measured_kib = max(values.values())
    return copy_bytes / measured_kib


def traffic(
    fetch_dir: str | Path,
    write_dir: str | Path,
    copy_fetch_dir: str | Path,
    copy_write_dir: str | Path,
    copy_bytes: int = COPY_CALIBRATION_BYTES,
    name_filter: str = "w4a16",
) -> dict:
    rs = copy_scale(copy_fetch_dir, "FETCH_SIZE", copy_bytes)
    ws = copy_scale(copy_write_dir, "WRITE_SIZE", copy_bytes)
    fetch = counter_by_grid(fetch_dir, "FETCH_SIZE", name_filter)
    write = counter_by_grid(write_dir, "WRITE_SIZE", name_filter)
    rows = {}
    for key in sorted(set(fetch) | set(write), key=lambda k: k[1]):
        f = fetch.get(key, 0.0) * rs
        w = write.get(key, 0.0) * ws
        rows[f"{key[0]} grid={key[1]}"] = {
            "fetch_kib_raw": fetch.get(key),
            "write_kib_raw": write.get(key),
            "read_bytes": round(f),
            "write_bytes": round(w),
            "hbm_bytes_per_launch": round(f + w),
        }
    return {"read_scale_bytes_per_kib": rs, "write_scale_bytes_per_kib": ws, "kernels": rows}


def _shape_row(rows: dict, threads: int, slice_cols: int | None,
               native: bool | None = None) -> tuple[str, dict] | None:
    """The kernel row of one bench shape: same grid and, when several kernels share the grid, the
    packet format (native-slab kernels, whatever their slice width: single slices, slice pairs
    and the stream schedule all carry "native" or "stream" in their names) or, for the
    reference-packet kernel, the slice width its template arguments carry as
    ", <cols>, (PacketFormat)"."""
    hits = [(k, v) for k, v in rows.items() if k.endswith(f" grid={threads}")]
    if len(hits) > 1 and native is not None:
        hits = [(k, v) for k, v in hits if (("native" in k or "stream" in k) == native)]
    if len(hits) > 1 and slice_cols is not None:
        hits = [(k, v) for k, v in hits if f", {slice_cols}, (PacketFormat)" in k]
    return hits[0] if len(hits) == 1 else None


def traffic_by_shape(result: dict, bench: dict) -> dict:
    """traffic() rows keyed by the bench line's shape names (per_shape workgroups x 256 threads,
    slice_cols), with the algorithmic bytes beside them."""
    out = {}
    native = bench.get("config", {}).get("packets", "native_sym") != "arc"
    for name, shape in bench["per_shape"].items():
        threads = int(shape["workgroups"]) * int(shape.get("threads_per_workgroup", 256))
        hit = _shape_row(result["kernels"], threads, shape.get("slice_cols"), native)
        if hit is None:
            continue
        kernel, row = hit
        out[name] = dict(row, kernel=kernel, grid_threads=threads,
                         algorithmic_bytes=int(shape["bytes"]),
                         traffic_over_algorithmic=round(row["hbm_bytes_per_launch"] / shape["bytes"], 4))
    return out


def _markdown_trace(rows: list[dict]) -> str:
    lines = [
        "| kernel | grid threads | workgroups | calls | avg us | median us | min us | max us |",
        "|---|---:|---:|---:|---:|---:|---:|---:|",
    ]
    for r in rows:
        lines.append(
            f"| `{r['kernel']}` | {r['grid_threads']} | {r['workgroups']} | {r['calls']} | "
            f"{r['avg_us']:.2f} | {r['median_us']:.2f} | {r['min_us']:.2f} | {r['max_us']:.2f} |"
        )
    return "\n".join(lines)


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = p.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("directory")
    t.add_argument("--filter", default="")
    t.add_argument("--split-us", type=float, default=None,
                   help="split (kernel, grid) rows whose dispatches fall on both sides of this "
                   "duration")
    c = sub.add_parser("traffic")
    c.add_argument("--fetch", required=True)
    c.add_argument("--write", required=True)
    c.add_argument("--copy-fetch", required=True)
    c.add_argument("--copy-write", required=True)
    c.add_argument("--copy-bytes", type=int, default=COPY_CALIBRATION_BYTES)
    c.add_argument("--filter", default="w4a16")
    c.add_argument("--bench-json", help="bench.py line of the profiled run: key rows by shape")
    args = p.parse_args(argv)
    if args.cmd == "trace":
        print(_markdown_trace(kernel_trace_by_grid(args.directory, args.filter, args.split_us)))
    else:
        result = traffic(args.fetch, args.write, args.copy_fetch, args.copy_write, args.copy_bytes,
                         args.filter)
        if args.bench_json:
            bench = json.loads(Path(args.bench_json).read_text().strip().splitlines()[-1])
            result = {
                "read_scale_bytes_per_kib": result["read_scale_bytes_per_kib"],
                "write_scale_bytes_per_kib": result["write_scale_bytes_per_kib"],
                bench["config"]["workload"]: traffic_by_shape(result, bench),
            }
        print(json.dumps(result, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
