"""Test configuration: import paths for the package (fast-kernels_amd/) and the oracle, the
``gpu`` marker, and shared fixtures."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

try:  # load PyTorch's HIP runtime before anything loads libfk_w4a16.so (one runtime per process)
    import torch  # noqa: F401
except ImportError:  # pragma: no cover
    pass

REPO_ROOT = Path(__file__).resolve().parent.parent
PKG_PARENT = REPO_ROOT / "fast-kernels_amd"
for p in (str(PKG_PARENT), str(REPO_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


@pytest.fixture(scope="session")
def project_dir() -> Path:
    return PKG_PARENT


@pytest.fixture(autouse=True)
def _chdir_project(monkeypatch: pytest.MonkeyPatch) -> None:
    # Suite paths in the CLI tests are relative to the project directory, as in the reference.
    monkeypatch.chdir(PKG_PARENT)


def gpu_available() -> bool:
    try:
        import torch
    except ImportError:
        return False
    return bool(torch.cuda.is_available())


os.environ.setdefault("PYTHONHASHSEED", "0")
