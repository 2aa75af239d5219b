from fast_kernels.benchmarking.runner import benchmark_suite, summarize_statuses, verify_suite
from fast_kernels.benchmarking.suites import load_suite

__all__ = ["benchmark_suite", "load_suite", "summarize_statuses", "verify_suite"]
