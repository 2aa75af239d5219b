"""Environment snapshot for ``fk env`` and run metadata (reference: src/fast_kernels/env.py:15-103),
reporting the ROCm tools (rocm-smi, hipcc) where the reference reports nvidia-smi and nvcc."""

from __future__ import annotations

import json
import os
import platform
import re
import shutil
import subprocess
import sys
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Any

from fast_kernels.native import native_build_info


@dataclass
class EnvironmentSnapshot:
    python_version: str
    platform: str
    machine: str
    git_sha: str | None
    git_dirty: bool
    native: dict[str, Any]
    rocm_smi: dict[str, str] | None
    hipcc_version: str | None
    torch_version: str | None
    cpu_cores: int
    nvidia_smi: dict[str, str] | None = None
    nvcc_version: str | None = None

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), indent=2, sort_keys=True)


def _run_capture(command: list[str], cwd: Path | None = None) -> str | None:
    if shutil.which(command[0]) is None:
        return None
    try:
        completed = subprocess.run(command, capture_output=True, check=False, cwd=cwd, text=True,
                                   timeout=30)
    except (OSError, subprocess.TimeoutExpired):
        return None
    if completed.returncode != 0:
        return None
    return completed.stdout.strip()


def _git_sha(repo: Path | None = None) -> str | None:
    return _run_capture(["git", "rev-parse", "--short", "HEAD"], cwd=repo)


def _git_dirty(repo: Path | None = None) -> bool:
    return bool(_run_capture(["git", "status", "--porcelain"], cwd=repo))


def _torch_version() -> str | None:
    try:
        import torch
    except ImportError:
        return None
    return str(torch.__version__)


def _rocm_smi() -> dict[str, str] | None:
    """GPU name and driver version from rocm-smi (first device), None without a GPU."""
    output = _run_capture(["rocm-smi", "--showproductname", "--showdriverversion", "--json"])
    if not output:
        return None
    try:
        payload = json.loads(output[output.index("{"):])
    except (ValueError, json.JSONDecodeError):
        return None
    info: dict[str, str] = {}
    for key, value in payload.items():
        if not isinstance(value, dict):
            continue
        if key.startswith("card") and "name" not in info:
            names = [value.get(k) for k in ("Card Series", "Card series", "Card Model", "Card SKU")]
            name = next((str(n) for n in names if n and str(n).strip() not in {"N/A", "0x0"}), None)
            if name:
                info["name"] = name
            gfx = value.get("GFX Version")
            if gfx:
                info["gfx_version"] = str(gfx)
        if key == "system" and "Driver version" in value:
            info["driver_version"] = str(value["Driver version"])
    return info or None


def _hipcc_version() -> str | None:
    output = _run_capture(["hipcc", "--version"])
    if output is None:
        return None
    match = re.search(r"HIP version:\s*(\S+)", output)
    return match.group(1) if match else output.splitlines()[0]


def _cpu_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover - non-Linux
        return os.cpu_count() or 1


def collect_environment(repo: Path | None = None) -> EnvironmentSnapshot:
    return EnvironmentSnapshot(
        python_version=sys.version.split()[0],
        platform=platform.platform(),
        machine=platform.machine(),
        git_sha=_git_sha(repo),
        git_dirty=_git_dirty(repo),
        native=native_build_info(),
        rocm_smi=_rocm_smi(),
        hipcc_version=_hipcc_version(),
        torch_version=_torch_version(),
        cpu_cores=_cpu_cores(),
    )
