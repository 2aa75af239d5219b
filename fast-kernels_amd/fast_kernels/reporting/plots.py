"""SVG plots of a result bundle, written directly as SVG text (no plotting library needed).

``status_counts.svg`` matches the reference's plot (src/fast_kernels/reporting/plots.py:15-30): one
bar per case status. ``hbm_bandwidth.svg`` adds effective HBM GB/s per timed case against the
MI355X peak.
"""

from __future__ import annotations

from collections import Counter
from pathlib import Path
from xml.sax.saxutils import escape

from fast_kernels.schemas import ResultBundle

_COLORS = ["#1f77b4", "#ff7f0e", "#2ca02c", "#d62728", "#9467bd", "#8c564b"]


def _bar_svg(title: str, labels: list[str], values: list[float], y_label: str,
             ref_line: float | None = None) -> str:
    width, height = 900, 480
    left, right, top, bottom = 70, 20, 50, 150
    plot_w, plot_h = width - left - right, height - top - bottom
    vmax = max([*values, ref_line or 0.0, 1e-9])
    n = max(len(values), 1)
    slot = plot_w / n
    bar_w = slot * 0.7
    parts = [
        f'<svg xmlns="http://www.w3.org/2000/svg" width="{width}" height="{height}" '
        f'viewBox="0 0 {width} {height}" font-family="sans-serif" font-size="11">',
        f'<text x="{width / 2}" y="25" text-anchor="middle" font-size="15">{escape(title)}</text>',
        f'<line x1="{left}" y1="{top + plot_h}" x2="{left + plot_w}" y2="{top + plot_h}" stroke="#333"/>',
        f'<line x1="{left}" y1="{top}" x2="{left}" y2="{top + plot_h}" stroke="#333"/>',
        f'<text x="15" y="{top + plot_h / 2}" transform="rotate(-90 15 {top + plot_h / 2})" '
        f'text-anchor="middle">{escape(y_label)}</text>',
    ]
    for i in range(5):
        v = vmax * i / 4
        y = top + plot_h - plot_h * i / 4
        parts.append(f'<line x1="{left}" y1="{y:.1f}" x2="{left + plot_w}" y2="{y:.1f}" stroke="#ddd"/>')
        parts.append(f'<text x="{left - 5}" y="{y + 4:.1f}" text-anchor="end">{v:.3g}</text>')
    for i, (label, value) in enumerate(zip(labels, values)):
        h = plot_h * value / vmax
        x = left + i * slot + (slot - bar_w) / 2
        y = top + plot_h - h
        color = _COLORS[i % len(_COLORS)]
        parts.append(f'<rect x="{x:.1f}" y="{y:.1f}" width="{bar_w:.1f}" height="{h:.1f}" fill="{color}"/>')
        parts.append(f'<text x="{x + bar_w / 2:.1f}" y="{y - 3:.1f}" text-anchor="middle">{value:.4g}</text>')
        tx = x + bar_w / 2
        ty = top + plot_h + 10
        parts.append(f'<text x="{tx:.1f}" y="{ty:.1f}" transform="rotate(45 {tx:.1f} {ty:.1f})">'
                     f'{escape(label)}</text>')
    if ref_line is not None:
        y = top + plot_h - plot_h * ref_line / vmax
        parts.append(f'<line x1="{left}" y1="{y:.1f}" x2="{left + plot_w}" y2="{y:.1f}" '
                     f'stroke="#d62728" stroke-dasharray="6,4"/>')
        parts.append(f'<text x="{left + plot_w}" y="{y - 4:.1f}" text-anchor="end" fill="#d62728">'
                     f'peak {ref_line:.4g}</text>')
    parts.append("</svg>")
    return "\n".join(parts) + "\n"


def render_plot(bundle: ResultBundle, destination: str | Path) -> Path:
    output_path = Path(destination)
    output_path.parent.mkdir(parents=True, exist_ok=True)
    counts = Counter(case.status for case in bundle.cases)
    labels = list(counts.keys())
    output_path.write_text(
        _bar_svg(f"{bundle.metadata.suite_id} status counts", labels,
                 [float(counts[label]) for label in labels], "cases"),
        encoding="utf-8",
    )
    return output_path


def render_bandwidth_plot(bundle: ResultBundle, destination: str | Path,
                          peak_gbs: float = 8000.0) -> Path | None:
    timed = [c for c in bundle.cases if c.status == "ok" and "hbm_gbs" in c.metrics]
    if not timed:
        return None
    output_path = Path(destination)
    output_path.parent.mkdir(parents=True, exist_ok=True)
    labels = [f"{c.subject_id.split('/')[-1]}:{c.shape_name}" for c in timed]
    output_path.write_text(
        _bar_svg(f"{bundle.metadata.suite_id} effective HBM GB/s", labels,
                 [c.metrics["hbm_gbs"] for c in timed], "GB/s", ref_line=peak_gbs),
        encoding="utf-8",
    )
    return output_path
