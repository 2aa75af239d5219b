"""Build the native W4A16 library and its Python binding, in-tree.

Outputs (next to the Python package, so they travel with the source tree):
  fast-kernels_amd/fast_kernels/libfk_w4a16.so   HIP kernels + C++ ops + the C ABI (fk_w4a16.h)
  fast-kernels_amd/fast_kernels/_native*.so      pybind11 module over the C ABI

Compiles for gfx950 only with hipcc; packed-fp32 instruction selection is disabled. Every call
recompiles (the driver uses a call as the "does it build" check).
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
OUT_DIR = PKG_ROOT / "fast_kernels"
BUILD_DIR = PKG_ROOT / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

LIB_SOURCES = [
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemv.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemv_native.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemv_stream.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemv_arc_stream.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemv_arc_quarter.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemv_fused.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemm_mfma.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_gemm_mfma_stream.hip",
    CSRC / "kernels" / "decode_quant_linear" / "w4a16_aux.hip",
    CSRC / "ops" / "decode_quant_linear" / "arc_w4a16_ops.cpp",
    CSRC / "ops" / "decode_quant_linear" / "w4a16_scratch.hip",
    CSRC / "capi" / "fk_w4a16_capi.cpp",
]

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{CSRC}",
    f"-I{CSRC / 'kernels' / 'decode_quant_linear'}",
    f"-I{REPO_ROOT / 'include'}",
]

LIB_NAME = "libfk_w4a16.so"


def hip_runtime_dir() -> Path:
    """Directory of the HIP runtime the library must share with its host process.

    A process may hold only one HIP runtime: PyTorch-ROCm wheels ship their own libamdhip64.so
    (and libhipblaslt.so) under torch/lib, and a second copy from /opt/rocm in the same process
    gives two runtimes whose streams and pointers are foreign to each other. So when torch is
    importable the library links against torch's copies (rpath to torch/lib); otherwise against
    /opt/rocm/lib.
    """
    try:
        import importlib.util

        spec = importlib.util.find_spec("torch")
        if spec is not None and spec.origin is not None:
            lib_dir = Path(spec.origin).parent / "lib"
            if (lib_dir / "libamdhip64.so").exists() and (lib_dir / "libhipblaslt.so").exists():
                return lib_dir
    except (ImportError, ValueError):
        pass
    return Path("/opt/rocm/lib")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}"
        )


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.name + ".o")
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    _run([HIPCC, *HIP_FLAGS, *lang, "-c", str(src), "-o", str(obj)])
    return obj


def build_library() -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(LIB_SOURCES))) as pool:
        objects = list(pool.map(_compile, LIB_SOURCES))
    lib = OUT_DIR / LIB_NAME
    tmp = BUILD_DIR / LIB_NAME
    rt = hip_runtime_dir()
    _run(
        [
            "g++",
            "-shared",
            "-fPIC",
            *map(str, objects),
            "-o",
            str(tmp),
            f"-L{rt}",
            "-l:libamdhip64.so",
            "-l:libhipblaslt.so",
            f"-Wl,-rpath,{rt}",
            "-Wl,--no-undefined",
        ]
    )
    os.replace(tmp, lib)
    return lib


def build_binding() -> Path:
    import pybind11

    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    target = OUT_DIR / f"_native{ext_suffix}"
    tmp = BUILD_DIR / target.name
    _run(
        [
            "g++",
            "-O2",
            "-std=c++17",
            "-fPIC",
            "-shared",
            "-fvisibility=hidden",
            f"-I{pybind11.get_include()}",
            f"-I{sysconfig.get_paths()['include']}",
            f"-I{REPO_ROOT / 'include'}",
            str(CSRC / "bindings" / "python_module.cpp"),
            "-o",
            str(tmp),
            f"-L{OUT_DIR}",
            "-lfk_w4a16",
            "-Wl,-rpath,$ORIGIN",
        ]
    )
    os.replace(tmp, target)
    return target


def build() -> list[Path]:
    return [build_library(), build_binding()]


if __name__ == "__main__":
    for path in build():
        print(path)
    sys.exit(0)
