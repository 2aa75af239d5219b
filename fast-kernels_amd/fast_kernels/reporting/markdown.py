"""summary.md of a result bundle.

Sections: the run header, the cases grouped per (dtype, layout, shape) with the kernels and
baselines of a shape side by side (device time, HBM bandwidth and its share of the MI355X peak,
speed-ups, and the measured HBM traffic when ``fk bench --counters`` recorded it), then the
cases that did not run with their reasons, and the run notes. The reference writes one flat
table (src/fast_kernels/reporting/markdown.py:16-79); the per-shape grouping makes a kernel's
bandwidth directly comparable with its baselines'.
"""

from __future__ import annotations

from collections import Counter, defaultdict

from fast_kernels.schemas import BenchmarkCase, ResultBundle


def _num(value: float | None, digits: int = 1) -> str:
    return "" if value is None else f"{value:.{digits}f}"


def _gpu_name(bundle: ResultBundle) -> str:
    meta = bundle.metadata
    smi = meta.rocm_smi or {}
    return smi.get("name") or smi.get("gfx_version") or (meta.nvidia_smi or {}).get("name") or "none"


def _header(bundle: ResultBundle) -> list[str]:
    meta = bundle.metadata
    counts = Counter(case.status for case in bundle.cases)
    status = ", ".join(f"{n} {s}" for s, n in sorted(counts.items()))
    return [
        f"# {meta.suite_id}",
        "",
        f"Run `{meta.run_id}` created `{meta.created_at}` at git `{meta.git_sha or 'uncommitted'}`, "
        f"Python `{meta.python_version}` on `{meta.platform}`, GPU `{_gpu_name(bundle)}`, native "
        f"backend available: `{meta.native.get('available', False)}`.",
        "",
        f"Cases: {status}.",
        "",
    ]


_COLUMNS = ("subject", "status", "device us", "p95 us", "wall us", "HBM GB/s", "% peak",
            "measured HBM / alg.", "speed-up", "max abs err")


def _case_row(case: BenchmarkCase) -> str:
    m = case.metrics
    speedup = ", ".join(f"{v:.2f}x vs `{b}`" for b, v in sorted(case.speedup_vs.items()))
    traffic = m.get("traffic_over_algorithmic")
    cells = (
        f"{case.subject_kind} `{case.subject_id}`",
        case.status,
        _num(case.device_latency_us_median, 2),
        _num(case.device_latency_us_p95, 2),
        _num(case.wall_latency_us_median or case.latency_us_median),
        _num(m.get("hbm_gbs")),
        _num(m.get("pct_hbm_peak")),
        "" if traffic is None else f"{traffic:.3f}",
        speedup,
        "" if m.get("max_abs_err") is None else f"{m['max_abs_err']:.3g}",
    )
    return "| " + " | ".join(cells) + " |"


def render_summary_markdown(bundle: ResultBundle) -> str:
    lines = _header(bundle)
    by_shape: dict[tuple[str, str, str], list[BenchmarkCase]] = defaultdict(list)
    for case in bundle.cases:
        by_shape[(case.dtype, case.layout, case.shape_name)].append(case)
    lines += ["## Results by shape", ""]
    for (dtype, layout, shape), cases in by_shape.items():
        dims = ", ".join(f"{k}={v}" for k, v in cases[0].dimensions.items())
        lines += [f"### {shape} ({dtype}, {layout}; {dims})", "",
                  "| " + " | ".join(_COLUMNS) + " |",
                  "|" + "|".join(" --- " if i < 2 else " ---: " for i in range(len(_COLUMNS))) + "|"]
        lines += [_case_row(c) for c in cases]
        lines.append("")
    not_run = [c for c in bundle.cases if c.status != "ok" and c.reason]
    if not_run:
        lines += ["## Cases that did not run", ""]
        lines += [f"- `{c.case_id}` ({c.status}): {c.reason}" for c in not_run]
        lines.append("")
    if bundle.metadata.notes:
        lines += ["## Notes", ""] + [f"- {note}" for note in bundle.metadata.notes] + [""]
    lines += ["## Case ids", ""] + [f"- `{c.case_id}`" for c in bundle.cases] + [""]
    return "\n".join(lines)
