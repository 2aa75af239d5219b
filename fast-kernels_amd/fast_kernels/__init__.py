"""fast-kernels for MI355X: the W4A16 decode-linear path on hand-written gfx950 HIP kernels."""

from fast_kernels.native import native_available, native_build_info

__version__ = "0.1.0"

__all__ = ["__version__", "native_available", "native_build_info"]
