"""Repository and result-root discovery (reference: src/fast_kernels/paths.py:6-18)."""

from __future__ import annotations

from pathlib import Path


def package_root() -> Path:
    return Path(__file__).resolve().parent


def project_root() -> Path:
    """The directory holding ``fast_kernels/``, ``csrc/`` and ``benchmarks/``."""
    return package_root().parent


def repo_root() -> Path:
    for candidate in package_root().parents:
        if (candidate / ".git").exists():
            return candidate
    return project_root()


def benchmarks_root() -> Path:
    return project_root() / "benchmarks"


def default_results_root() -> Path:
    return repo_root() / "results"
