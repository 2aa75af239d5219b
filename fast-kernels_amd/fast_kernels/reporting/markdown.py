"""summary.md of a result bundle (reference layout: src/fast_kernels/reporting/markdown.py:16-79)."""

from __future__ import annotations

from collections import Counter

from fast_kernels.schemas import ResultBundle


def _fmt(value: float | None, digits: int = 1) -> str:
    if value is None:
        return ""
    return f"{value:.{digits}f}"


def render_summary_markdown(bundle: ResultBundle) -> str:
    meta = bundle.metadata
    status_counts = Counter(case.status for case in bundle.cases)
    smi = meta.rocm_smi or {}
    gpu = smi.get("name") or smi.get("gfx_version") or (meta.nvidia_smi or {}).get("name") or "none"
    lines = [
        f"# {meta.suite_id}",
        "",
        f"- Run ID: `{meta.run_id}`",
        f"- Created: `{meta.created_at}`",
        f"- Git SHA: `{meta.git_sha or 'uncommitted'}`",
        f"- Python: `{meta.python_version}`",
        f"- Platform: `{meta.platform}`",
        f"- GPU: `{gpu}`",
        f"- Native backend available: `{meta.native.get('available', False)}`",
        "",
        "## Status Summary",
        "",
        "| status | count |",
        "| --- | ---: |",
    ]
    for status, count in sorted(status_counts.items()):
        lines.append(f"| {status} | {count} |")
    lines += ["", "## Notes", ""]
    lines += [f"- {note}" for note in meta.notes]
    lines += [
        "",
        "## Cases",
        "",
        "| case | subject | dtype | layout | shape | status | wall us | device us | p95 us | "
        "decode tok/s | HBM GB/s | % peak | speedup | metrics |",
        "| --- | --- | --- | --- | --- | --- | ---: | ---: | ---: | ---: | ---: | ---: | --- | --- |",
    ]
    for case in bundle.cases:
        speedup = ", ".join(f"{b}={v:.2f}x" for b, v in sorted(case.speedup_vs.items()))
        extra = {k: v for k, v in case.metrics.items() if k not in {"hbm_gbs", "pct_hbm_peak"}}
        metrics = ", ".join(f"{k}={v:.4g}" for k, v in sorted(extra.items()))
        lines.append(
            f"| `{case.case_id}` | `{case.subject_id}` | `{case.dtype}` | `{case.layout}` | "
            f"`{case.shape_name}` | `{case.status}` | "
            f"{_fmt(case.wall_latency_us_median or case.latency_us_median)} | "
            f"{_fmt(case.device_latency_us_median, 2)} | "
            f"{_fmt(case.wall_latency_us_p95 or case.latency_us_p95)} | "
            f"{_fmt(case.decode_tokens_per_second or case.throughput)} | "
            f"{_fmt(case.metrics.get('hbm_gbs'))} | {_fmt(case.metrics.get('pct_hbm_peak'))} | "
            f"{speedup} | {metrics} |"
        )
        if case.reason and case.status != "ok":
            lines.append(f"|  | reason: {case.reason.replace('|', '/')} |  |  |  |  |  |  |  |  |  |  |  |  |")
    lines.append("")
    return "\n".join(lines)
