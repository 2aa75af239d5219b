from fast_kernels.reporting.artifacts import load_result_bundle, write_result_bundle
from fast_kernels.reporting.markdown import render_summary_markdown
from fast_kernels.reporting.plots import render_bandwidth_plot, render_plot

__all__ = [
    "load_result_bundle",
    "render_bandwidth_plot",
    "render_plot",
    "render_summary_markdown",
    "write_result_bundle",
]
