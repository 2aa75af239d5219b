"""Seeded synthetic W4A16 inputs (host, numpy) shared by the suite runner, tests and bench.

Recipe (the benchmark configuration's, a variant of the reference's _make_case_inputs,
src/fast_kernels/benchmarking/decode_linear_w4a16.py:152-174):
  codes    U{0..15}, drawn as uniform bytes of q_u8 [N, K/2] (two independent nibbles per byte)
  alpha    fp16(U[0.001, 0.02])                     [N, K/G]
  zero pt  symmetric: 8 for every group, beta = -8*alpha (exact in fp16)
           asymmetric: U{0..15} per group, beta = -half_rn(alpha * zp)
           (decode_linear_w4a16.py:172-173)
  x        N(0, 1) rounded to fp16 or bf16          [M, K]
Seed: the reference's case seed (decode_linear_w4a16.py:148-149) unless one is given.
All arrays are numpy; 16-bit floats are returned as uint16 bit patterns (bf16 has no numpy dtype).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


def seed_for_case(batch: int, n: int, k: int, group_size: int) -> int:
    return (batch * 1_000_003 + n * 1009 + k * 101 + group_size) % (2**31 - 1)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, as uint16 bits (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return b.view(np.float16).astype(np.float32)


@dataclass
class W4A16Case:
    x: np.ndarray       # uint16 bits [M, K]
    q_u8: np.ndarray    # uint8 [N, K/2]
    alpha: np.ndarray   # uint16 (fp16 bits) [N, NG]
    beta: np.ndarray    # uint16 (fp16 bits) [N, NG]
    zero_points: np.ndarray  # uint8 [N, NG]
    act: str            # "f16" or "bf16"
    batch: int
    n: int
    k: int
    group_size: int
    seed: int

    def x_f32(self) -> np.ndarray:
        return f16_bits_to_f32(self.x) if self.act == "f16" else bf16_bits_to_f32(self.x)


def make_case(
    batch: int,
    n: int,
    k: int,
    group_size: int,
    *,
    act: str = "f16",
    asymmetric: bool = False,
    seed: int | None = None,
    recipe: str = "baseline",
) -> W4A16Case:
    """recipe "baseline": the distributions in this module's docstring. recipe "reference": the
    reference suite's own distributions (decode_linear_w4a16.py:152-174): x = 0.25 N(0, 1),
    alpha U[0.02, 0.2], zero points U{0..15} (always asymmetric); the values differ from the
    reference's (it draws them from torch's CUDA generator), the distributions do not."""
    if act not in {"f16", "bf16"}:
        raise ValueError("act must be 'f16' or 'bf16'")
    if recipe not in {"baseline", "reference"}:
        raise ValueError("recipe must be 'baseline' or 'reference'")
    alpha_lo, alpha_hi, x_scale = (0.001, 0.02, 1.0) if recipe == "baseline" else (0.02, 0.2, 0.25)
    if recipe == "reference":
        asymmetric = True
    if k % group_size != 0 or k % 2 != 0:
        raise ValueError("k must be a multiple of group_size")
    if seed is None:
        seed = seed_for_case(batch, n, k, group_size)
    rng = np.random.default_rng(seed)
    ng = k // group_size
    q_u8 = rng.integers(0, 256, size=(n, k // 2), dtype=np.uint8)
    alpha16 = rng.uniform(alpha_lo, alpha_hi, size=(n, ng)).astype(np.float16)
    if asymmetric:
        zp = rng.integers(0, 16, size=(n, ng), dtype=np.uint8)
    else:
        zp = np.full((n, ng), 8, dtype=np.uint8)
    # half_rn(alpha * zp): the fp32 product of an fp16 and a small integer is exact
    beta16 = (-(alpha16.astype(np.float32) * zp.astype(np.float32))).astype(np.float16)
    x32 = rng.standard_normal(size=(batch, k), dtype=np.float32)
    if x_scale != 1.0:
        x32 *= np.float32(x_scale)
    x = x32.astype(np.float16).view(np.uint16) if act == "f16" else f32_to_bf16_bits(x32)
    return W4A16Case(
        x=np.ascontiguousarray(x),
        q_u8=q_u8,
        alpha=alpha16.view(np.uint16),
        beta=beta16.view(np.uint16),
        zero_points=zp,
        act=act,
        batch=batch,
        n=n,
        k=k,
        group_size=group_size,
        seed=seed,
    )


def algorithmic_bytes(
    batch: int, n: int, k: int, group_size: int, *, asymmetric: bool = False
) -> int:
    """Bytes a W4A16 GEMV must move: int4 codes + fp16 scales (+ int4 zero points when
    asymmetric) + activations + outputs. The packet format's fp16 beta is not credited."""
    ng = k // group_size
    b = n * k // 2 + n * ng * 2 + batch * k * 2 + batch * n * 2
    if asymmetric:
        b += n * ng // 2
    return b
