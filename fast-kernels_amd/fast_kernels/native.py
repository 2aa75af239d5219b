"""Loader for the compiled extension ``fast_kernels._native`` (pybind11 over libfk_w4a16.so).

Mirrors the reference loader (src/fast_kernels/native.py:8-37): importing never raises, and
``native_module()`` raises RuntimeError with the import error when the extension is missing, so
every op fails loudly instead of falling back to anything else.
"""

from __future__ import annotations

from importlib import import_module
from types import ModuleType
from typing import Any

_native: ModuleType | None
_native_import_error: ImportError | None

# One process may hold only one HIP runtime. PyTorch-ROCm ships its own libamdhip64 /
# libhipblaslt / libhsa-runtime64 (same sonames as /opt/rocm's); loading torch first makes the
# extension's dependencies bind to those already-loaded copies instead of pulling in a second
# runtime from /opt/rocm, whose streams and device pointers would be foreign to torch's.
try:
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - the C ABI itself does not need torch
    pass

try:
    _native = import_module("fast_kernels._native")
except ImportError as exc:  # pragma: no cover - exercised only when the build is missing
    _native = None
    _native_import_error = exc
else:
    _native_import_error = None


def native_available() -> bool:
    return _native is not None


def native_module() -> ModuleType:
    if _native is None:
        raise RuntimeError(
            f"native module unavailable: {_native_import_error}. "
            "Build it with `python __graft_entry__.py` or `python fast-kernels_amd/build_native.py`."
        )
    return _native


def native_build_info() -> dict[str, Any]:
    if _native is None:
        return {
            "available": False,
            "error": str(_native_import_error),
        }
    info = dict(_native.build_info())
    info["available"] = True
    return info
