"""The CMake build (fast-kernels_amd/CMakeLists.txt): a host-only configure + build
(FK_ENABLE_HIP=OFF) yields a stub libfk_w4a16.so with every entry point of include/fk_w4a16.h,
each failing with FK_ERR_RUNTIME, and a _native module reporting compiled_with_hip False; the
HIP configure lists the same sources as build_native.py."""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "fast-kernels_amd"
HEADER = REPO / "include" / "fk_w4a16.h"
FK_ERR_RUNTIME = 2

pytestmark = pytest.mark.skipif(shutil.which("cmake") is None, reason="cmake not on PATH")


def _declared() -> list[str]:
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(fk_\w+)\s*\(", HEADER.read_text(),
                                 re.M)))


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=600, cwd=cwd)
    assert proc.returncode == 0, f"{' '.join(cmd)}\n{proc.stdout[-3000:]}\n{proc.stderr[-3000:]}"


@pytest.fixture(scope="module")
def cpu_build(tmp_path_factory: pytest.TempPathFactory) -> Path:
    build = tmp_path_factory.mktemp("cmake-cpu")
    gen = ["-G", "Ninja"] if shutil.which("ninja") else []
    _run(["cmake", "-S", str(PKG), "-B", str(build), *gen, "-DFK_ENABLE_HIP=OFF",
          "-DCMAKE_BUILD_TYPE=Release", f"-DPython_EXECUTABLE={sys.executable}"])
    _run(["cmake", "--build", str(build), "-j", "4"])
    return build


def test_stub_library_exports_every_declared_entry_point(cpu_build: Path) -> None:
    lib = ctypes.CDLL(str(cpu_build / "libfk_w4a16.so"))
    for name in _declared():
        assert hasattr(lib, name), name
    lib.fk_last_error.restype = ctypes.c_char_p
    lib.fk_build_info.restype = ctypes.c_char_p
    assert b"cpu-only" in lib.fk_build_info()
    status = lib.fk_arc_w4a16_forward(None, None, None, None, 1, 32, 128, 128, 2112, None)
    assert status == FK_ERR_RUNTIME
    assert b"FK_ENABLE_HIP=OFF" in lib.fk_last_error()


def test_stub_module_reports_no_hip(cpu_build: Path) -> None:
    code = ("import sys; sys.path.insert(0, sys.argv[1]); import _native; info = _native.build_info(); "
            "assert info['compiled_with_hip'] is False, info\n"
            "try:\n"
            "    _native.arc_w4a16_forward(0, 0, 0, 0, batch=1, n=32, k=128, group_size=128, "
            "packet_stride_bytes=2112, stream_ptr=0)\n"
            "except RuntimeError as e:\n"
            "    assert 'FK_ENABLE_HIP=OFF' in str(e)\n"
            "else:\n"
            "    raise AssertionError('stub call did not raise')\n")
    _run([sys.executable, "-c", code, str(cpu_build)])


def test_hip_sources_match_in_tree_build() -> None:
    sys.path.insert(0, str(PKG))
    try:
        import build_native
    finally:
        sys.path.pop(0)
    text = (PKG / "CMakeLists.txt").read_text()
    listed = {Path(m).name for m in re.findall(r"\$\{FK_(?:KERNEL_DIR|CSRC)\}/(\S+\.(?:hip|cpp))", text)}
    listed.discard("fk_w4a16_stub.cpp")
    listed.discard("python_module.cpp")
    assert listed == {p.name for p in build_native.LIB_SOURCES}
    assert "-packed-fp32-ops" in text and "gfx950" in text
