"""HBM traffic of benchmark cases, measured with rocprofv3 (``fk bench --counters``).

For every kernel case of a decode-linear suite that ran, the case is rebuilt in a child process
(``launch_kernel_case``: the timed run's inputs and rotated weight copies) and its kernel launched
LAUNCHES times under ``rocprofv3 --pmc FETCH_SIZE``, then again under ``--pmc WRITE_SIZE`` (one
counter per run: the counter blocks are small, and a request rocprofv3 cannot collect in one pass
hangs it). The mean counter value over the W4A16 kernel's dispatches, scaled by what the same
counter reports for a plain 256 MiB device-to-device copy (bytes per counter unit), is the HBM
traffic of one launch. Recorded in the case metrics:

  hbm_read_bytes_measured, hbm_write_bytes_measured, hbm_bytes_measured, and
  traffic_over_algorithmic = hbm_bytes_measured / algorithmic_bytes

(traffic well above the algorithmic bytes means bytes read twice). The profiled program is the
Python interpreter itself, placed right after ``--``, so no launcher sits between rocprofv3's
preloaded library and the process that uses the GPU.

Child commands (run by the parent under rocprofv3; usable by hand):
  python -m fast_kernels.benchmarking.counters copy
  python -m fast_kernels.benchmarking.counters case SUITE CASE_ID [--launches N]
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

from fast_kernels.benchmarking.rocprof import COPY_CALIBRATION_BYTES, copy_scale, counter_by_grid
from fast_kernels.schemas import BenchmarkCase

COUNTERS = ("FETCH_SIZE", "WRITE_SIZE")
LAUNCHES = 20
CHILD_TIMEOUT_S = 180
KERNEL_NAME_FILTERS = ("w4a16_gemv", "w4a16_gemm")


def _rocprof() -> str | None:
    found = shutil.which("rocprofv3")
    if found:
        return found
    fallback = Path("/opt/rocm/bin/rocprofv3")
    return str(fallback) if fallback.exists() else None


def _profile(rocprof: str, counter: str, child_args: list[str], out_dir: Path) -> Path:
    cmd = [rocprof, "--pmc", counter, "--output-format", "csv", "-d", str(out_dir), "-o", "run",
           "--", sys.executable, "-m", "fast_kernels.benchmarking.counters", *child_args]
    # The child runs from the scratch directory, so it finds this package through PYTHONPATH.
    pkg_parent = str(Path(__file__).resolve().parents[2])
    path = os.pathsep.join(p for p in (pkg_parent, os.environ.get("PYTHONPATH", "")) if p)
    env = dict(os.environ, TMPDIR=str(out_dir.parent), PYTHONPATH=path)
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=CHILD_TIMEOUT_S, env=env,
                          cwd=str(out_dir.parent))
    if proc.returncode != 0:
        tail = (proc.stdout + proc.stderr).strip().splitlines()[-5:]
        raise RuntimeError(f"rocprofv3 --pmc {counter} failed ({proc.returncode}): " + " | ".join(tail))
    return out_dir


def _kernel_counter(directory: Path, counter: str) -> float | None:
    """Mean counter value per dispatch of the case's W4A16 kernel (the grid with most dispatches)."""
    best: tuple[int, float] | None = None
    for name_filter in KERNEL_NAME_FILTERS:
        try:
            groups = counter_by_grid(directory, counter, name_filter, with_counts=True)
        except FileNotFoundError:
            return None
        for _, (mean, count) in groups.items():
            if best is None or count > best[0]:
                best = (count, mean)
    return None if best is None else best[1]


def add_traffic_metrics(suite_path: Path, cases: list[BenchmarkCase]) -> list[str]:
    """Measures every ok kernel case of the suite and adds the traffic metrics in place; returns
    notes for the run metadata (what was measured, or why nothing was)."""
    from fast_kernels.benchmarking.suites import load_suite

    suite_path = Path(suite_path).resolve()
    suite = load_suite(suite_path)
    if suite.family != "decode_quant_linear":
        return [f"--counters: no traffic measurement for suite family {suite.family!r}."]
    rocprof = _rocprof()
    if rocprof is None:
        return ["--counters: rocprofv3 not found; no traffic measured."]
    targets = [c for c in cases if c.subject_kind == "kernel" and c.status == "ok"]
    notes = []
    with tempfile.TemporaryDirectory(prefix="fk-counters-") as tmp:
        root = Path(tmp)
        scale = {}
        for counter in COUNTERS:
            d = _profile(rocprof, counter, ["copy"], root / f"copy-{counter}")
            scale[counter] = copy_scale(d, counter, COPY_CALIBRATION_BYTES)
        for i, case in enumerate(targets):
            print(f"[fk bench --counters] {i + 1}/{len(targets)} {case.case_id}", file=sys.stderr,
                  flush=True)
            raw = {}
            for counter in COUNTERS:
                d = _profile(rocprof, counter, ["case", str(suite_path), case.case_id],
                             root / f"case{i}-{counter}")
                raw[counter] = _kernel_counter(d, counter)
            if raw["FETCH_SIZE"] is None or raw["WRITE_SIZE"] is None:
                notes.append(f"--counters: no W4A16 kernel dispatch in {case.case_id} "
                             "(a vendor-library path); no traffic recorded.")
                continue
            read = raw["FETCH_SIZE"] * scale["FETCH_SIZE"]
            write = raw["WRITE_SIZE"] * scale["WRITE_SIZE"]
            case.metrics["hbm_read_bytes_measured"] = read
            case.metrics["hbm_write_bytes_measured"] = write
            case.metrics["hbm_bytes_measured"] = read + write
            alg = case.metrics.get("algorithmic_bytes")
            if alg:
                case.metrics["traffic_over_algorithmic"] = (read + write) / alg
    notes.insert(0, f"--counters: rocprofv3 FETCH_SIZE / WRITE_SIZE over {LAUNCHES} launches per "
                    f"kernel case ({len(targets)} cases), scaled by a {COPY_CALIBRATION_BYTES >> 20} "
                    f"MiB copy: {scale['FETCH_SIZE']:.1f} and {scale['WRITE_SIZE']:.1f} bytes per "
                    "counter unit.")
    return notes


def _copy_calibration() -> None:
    import torch

    src = torch.empty(COPY_CALIBRATION_BYTES, device="cuda", dtype=torch.uint8).random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description="Children of fk bench --counters.")
    sub = parser.add_subparsers(dest="what", required=True)
    sub.add_parser("copy", help="a 256 MiB device-to-device copy, 10 times")
    case = sub.add_parser("case", help="one kernel case of a suite, LAUNCHES launches")
    case.add_argument("suite", type=Path)
    case.add_argument("case_id")
    case.add_argument("--launches", type=int, default=LAUNCHES)
    args = parser.parse_args(argv)
    if args.what == "copy":
        _copy_calibration()
        return 0
    from fast_kernels.benchmarking.decode_linear_w4a16 import launch_kernel_case
    from fast_kernels.benchmarking.suites import load_suite

    launch_kernel_case(load_suite(args.suite), args.case_id, args.launches)
    return 0


if __name__ == "__main__":
    sys.exit(main())
