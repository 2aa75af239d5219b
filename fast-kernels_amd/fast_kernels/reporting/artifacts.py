"""Result-bundle files of a run directory (reference: src/fast_kernels/reporting/artifacts.py:14-77):
metadata.json, results.json, results.csv, summary.md, plots/status_counts.svg, and
plots/hbm_bandwidth.svg when cases carry HBM figures."""

from __future__ import annotations

import csv
import json
from pathlib import Path
from typing import Any

from fast_kernels.reporting.markdown import render_summary_markdown
from fast_kernels.reporting.plots import render_bandwidth_plot, render_plot
from fast_kernels.schemas import BenchmarkCase, ResultBundle

_CSV_FIELDS = (
    "case_id",
    "subject_kind",
    "subject_id",
    "dtype",
    "layout",
    "shape_name",
    "status",
    "latency_us_median",
    "latency_us_p95",
    "wall_latency_us_median",
    "wall_latency_us_p95",
    "device_latency_us_median",
    "device_latency_us_p95",
    "throughput",
    "decode_tokens_per_second",
    "context_tokens_per_second",
    "effective_kv_gib_per_second",
    "reason",
)


def _case_to_row(case: BenchmarkCase) -> dict[str, Any]:
    row: dict[str, Any] = {name: getattr(case, name) for name in _CSV_FIELDS}
    row["speedup_vs"] = json.dumps(case.speedup_vs, sort_keys=True)
    row["metrics"] = json.dumps(case.metrics, sort_keys=True)
    row["dimensions"] = json.dumps(case.dimensions, sort_keys=True)
    for key in ("m", "n", "k", "batch"):
        row[key] = case.dimensions.get(key)
    return row


def load_result_bundle(run_dir: str | Path) -> ResultBundle:
    payload = json.loads((Path(run_dir) / "results.json").read_text(encoding="utf-8"))
    return ResultBundle.model_validate(payload)


def write_result_bundle(run_dir: str | Path, bundle: ResultBundle) -> None:
    destination = Path(run_dir)
    plots_dir = destination / "plots"
    plots_dir.mkdir(parents=True, exist_ok=True)
    (destination / "metadata.json").write_text(
        json.dumps(bundle.metadata.model_dump(mode="json"), indent=2, sort_keys=True),
        encoding="utf-8",
    )
    (destination / "results.json").write_text(
        json.dumps(bundle.model_dump(mode="json"), indent=2, sort_keys=True), encoding="utf-8"
    )
    with (destination / "results.csv").open("w", encoding="utf-8", newline="") as handle:
        if bundle.cases:
            rows = [_case_to_row(case) for case in bundle.cases]
            writer = csv.DictWriter(handle, fieldnames=list(rows[0].keys()))
            writer.writeheader()
            writer.writerows(rows)
    (destination / "summary.md").write_text(render_summary_markdown(bundle), encoding="utf-8")
    render_plot(bundle, plots_dir / "status_counts.svg")
    render_bandwidth_plot(bundle, plots_dir / "hbm_bandwidth.svg")
