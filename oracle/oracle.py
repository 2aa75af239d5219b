"""ctypes front end of the C oracle (w4a16_oracle.c). TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module; the
product never does. See w4a16_oracle.c for the reference lines each function restates.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle_w4a16.so"

_lib: ctypes.CDLL | None = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "-B", "liboracle_w4a16.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I = ctypes.c_int
        L.fko_f32_to_f16_bits.argtypes = [ctypes.c_float]
        L.fko_f32_to_f16_bits.restype = ctypes.c_uint16
        L.fko_f16_bits_to_f32.argtypes = [ctypes.c_uint16]
        L.fko_f16_bits_to_f32.restype = ctypes.c_float
        L.fko_f32_to_bf16_bits.argtypes = [ctypes.c_float]
        L.fko_f32_to_bf16_bits.restype = ctypes.c_uint16
        L.fko_dequant.argtypes = [P, P, P, P, I, I, I]
        L.fko_pack_packets.argtypes = [P, P, P, P, I, I, I]
        L.fko_dequant_packets.argtypes = [P, P, I, I, I]
        L.fko_group_sums.argtypes = [P, P, I, I, I, I]
        L.fko_gemv.argtypes = [P, P, P, P, P, P, I, I, I, I, I]
        L.fko_gemv_f32.argtypes = [P, P, P, P, P, I, I, I, I, I]
        L.fko_reduce_partials.argtypes = [P, P, I, I, I]
        L.fko_packet_stride_bytes.argtypes = [I]
        L.fko_packet_stride_bytes.restype = ctypes.c_size_t
        L.fko_max_threads.restype = I
        L.fko_set_threads.argtypes = [I]
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f32_to_f16_bits(v: float) -> int:
    return int(lib().fko_f32_to_f16_bits(v))


def f32_to_f16_bits_array(a: np.ndarray) -> np.ndarray:
    f = lib().fko_f32_to_f16_bits
    flat = np.ascontiguousarray(a, dtype=np.float32).ravel()
    return np.array([f(float(v)) for v in flat], dtype=np.uint16).reshape(a.shape)


def dequant(q_u8: np.ndarray, alpha: np.ndarray, beta: np.ndarray, group_size: int) -> np.ndarray:
    n, half_k = q_u8.shape
    k = half_k * 2
    out = np.empty((n, k), dtype=np.uint16)
    lib().fko_dequant(_ptr(q_u8), _ptr(alpha), _ptr(beta), _ptr(out), n, k, group_size)
    return out


def packet_stride_bytes(group_size: int) -> int:
    return int(lib().fko_packet_stride_bytes(group_size))


def pack_packets(q_u8: np.ndarray, alpha: np.ndarray, beta: np.ndarray, group_size: int) -> np.ndarray:
    n, half_k = q_u8.shape
    k = half_k * 2
    rows = (n // 128) * (k // group_size)
    out = np.zeros((rows, packet_stride_bytes(group_size)), dtype=np.uint8)
    lib().fko_pack_packets(_ptr(q_u8), _ptr(alpha), _ptr(beta), _ptr(out), n, k, group_size)
    return out


def dequant_packets(packets: np.ndarray, n: int, k: int, group_size: int) -> np.ndarray:
    out = np.empty((n, k), dtype=np.uint16)
    lib().fko_dequant_packets(_ptr(packets), _ptr(out), n, k, group_size)
    return out


def group_sums(x_bits: np.ndarray, group_size: int, act: str = "f16") -> np.ndarray:
    batch, k = x_bits.shape
    out = np.empty((batch, k // group_size), dtype=np.float32)
    lib().fko_group_sums(_ptr(x_bits), _ptr(out), batch, k, group_size, 1 if act == "bf16" else 0)
    return out


def gemv(
    x_bits: np.ndarray,
    q_u8: np.ndarray,
    alpha: np.ndarray,
    beta: np.ndarray,
    group_size: int,
    act: str = "f16",
) -> tuple[np.ndarray, np.ndarray]:
    """Returns (y bits in the activation dtype [M, N], unrounded fp32 y [M, N])."""
    batch, k = x_bits.shape
    n = q_u8.shape[0]
    out = np.empty((batch, n), dtype=np.uint16)
    out32 = np.empty((batch, n), dtype=np.float32)
    lib().fko_gemv(
        _ptr(np.ascontiguousarray(x_bits)),
        _ptr(q_u8),
        _ptr(alpha),
        _ptr(beta),
        _ptr(out),
        _ptr(out32),
        batch,
        n,
        k,
        group_size,
        1 if act == "bf16" else 0,
    )
    return out, out32


def gemv_f32(
    x_bits: np.ndarray,
    q_u8: np.ndarray,
    alpha: np.ndarray,
    beta: np.ndarray,
    group_size: int,
    act: str = "f16",
) -> np.ndarray:
    """gemv with fp32 accumulation (the reference's arithmetic; the CPU baseline). Returns the
    output bits [M, N] in the activation dtype."""
    batch, k = x_bits.shape
    n = q_u8.shape[0]
    out = np.empty((batch, n), dtype=np.uint16)
    lib().fko_gemv_f32(
        _ptr(np.ascontiguousarray(x_bits)), _ptr(q_u8), _ptr(alpha), _ptr(beta), _ptr(out), batch,
        n, k, group_size, 1 if act == "bf16" else 0,
    )
    return out


def reduce_partials(partials: np.ndarray) -> np.ndarray:
    splits, batch, n = partials.shape
    out = np.empty((batch, n), dtype=np.uint16)
    lib().fko_reduce_partials(_ptr(np.ascontiguousarray(partials, dtype=np.float32)), _ptr(out), batch, n, splits)
    return out


def set_threads(threads: int) -> None:
    lib().fko_set_threads(threads)


def max_threads() -> int:
    return int(lib().fko_max_threads())
