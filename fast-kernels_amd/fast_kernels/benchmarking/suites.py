"""Suite loading (reference: src/fast_kernels/benchmarking/suites.py:1-13). Python 3.10 has no
tomllib; tomli is the same parser under its original name."""

from __future__ import annotations

from pathlib import Path

try:
    import tomllib
except ModuleNotFoundError:  # Python < 3.11
    import tomli as tomllib

from fast_kernels.schemas import BenchmarkSuite


def load_suite(path: str | Path) -> BenchmarkSuite:
    with Path(path).open("rb") as handle:
        payload = tomllib.load(handle)
    return BenchmarkSuite.model_validate(payload)
