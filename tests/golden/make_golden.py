"""Writes the W4A16 golden vectors in this directory (w4a16_golden.npz).

Two kinds of case:
  * "kat_*": known-answer cases whose expected outputs are computed here with exact integer
    arithmetic in pure Python, independent of the C oracle (alpha = 2^-e, beta = -8*alpha,
    x in {-2..2}, codes (n*7 + k*3) % 16); every value is exact in fp32 and in fp16, so dequant
    and GEMV have one right answer.
  * "rnd_*": seeded cases from fast_kernels.benchmarking.inputs.make_case with the C oracle's
    outputs (SHA-256 of the dequantized fp16 weights and of the packets, dequant row 0, group
    sums, y bits and unrounded fp32 y). They fix the oracle's behaviour across changes and give
    the GPU tests a frozen target.

Run from the repository root:  python tests/golden/make_golden.py
The reference publishes no golden vectors for this path, so none are copied.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "fast-kernels_amd"))
sys.path.insert(0, str(ROOT))

KAT_CASES = [
    # name, batch, n, k, group_size, scale exponent
    ("kat_m1_g64", 1, 128, 128, 64, 4),
    ("kat_m3_g128", 3, 256, 256, 128, 6),
]

RND_CASES = [
    # name, batch, n, k, group_size, act, asymmetric
    ("rnd_m1_g128_f16", 1, 128, 512, 128, "f16", False),
    ("rnd_m2_g64_f16_asym", 2, 128, 512, 64, "f16", True),
    ("rnd_m1_g128_bf16", 1, 128, 512, 128, "bf16", False),
    ("rnd_m4_g64_bf16_asym", 4, 128, 256, 64, "bf16", True),
]


def kat_case(batch: int, n: int, k: int, g: int, e: int) -> dict:
    """Exact integer known answer: W[n,k] = 2^-e * (q - 8), y[m,n] = 2^-e * sum (q-8) * x."""
    ng = k // g
    codes = [[(r * 7 + c * 3) % 16 for c in range(k)] for r in range(n)]
    q_u8 = np.zeros((n, k // 2), dtype=np.uint8)
    for r in range(n):
        for b in range(k // 2):
            q_u8[r, b] = codes[r][2 * b] | (codes[r][2 * b + 1] << 4)
    alpha = np.full((n, ng), 2.0 ** -e, dtype=np.float16).view(np.uint16)
    beta = np.full((n, ng), -8.0 * 2.0 ** -e, dtype=np.float16).view(np.uint16)
    xi = [[((m * 5 + c) % 5) - 2 for c in range(k)] for m in range(batch)]
    x = np.array(xi, dtype=np.float16).view(np.uint16)
    w_exact = np.array([[(codes[r][c] - 8) * 2.0 ** -e for c in range(k)] for r in range(n)])
    y = []
    for m in range(batch):
        row = []
        for r in range(n):
            acc = sum((codes[r][c] - 8) * xi[m][c] for c in range(k))  # exact integer
            row.append(acc * 2.0 ** -e)
        y.append(row)
    y = np.array(y)
    assert np.all(np.abs(y) < 2048), "known answers must be exact in fp16"
    return {
        "x": x,
        "q_u8": q_u8,
        "alpha": alpha,
        "beta": beta,
        "dequant": w_exact.astype(np.float16).view(np.uint16),
        "y": y.astype(np.float16).view(np.uint16),
        "meta": np.array([batch, n, k, g, 0, 0], dtype=np.int64),
    }


def sha256(a: np.ndarray) -> np.ndarray:
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest(), dtype=np.uint8)


def rnd_case(batch: int, n: int, k: int, g: int, act: str, asym: bool) -> dict:
    from fast_kernels.benchmarking.inputs import make_case
    from oracle import oracle

    c = make_case(batch, n, k, g, act=act, asymmetric=asym)
    y, y32 = oracle.gemv(c.x, c.q_u8, c.alpha, c.beta, g, act)
    packets = oracle.pack_packets(c.q_u8, c.alpha, c.beta, g)
    w = oracle.dequant(c.q_u8, c.alpha, c.beta, g)
    return {
        "x": c.x,
        "q_u8": c.q_u8,
        "alpha": c.alpha,
        "beta": c.beta,
        "dequant_sha256": sha256(w),
        "dequant_row0": w[0],
        "packets_sha256": sha256(packets),
        "group_sums": oracle.group_sums(c.x, g, act),
        "y": y,
        "y_f32": y32,
        "meta": np.array([batch, n, k, g, 1 if act == "bf16" else 0, 1 if asym else 0], dtype=np.int64),
    }


def main() -> int:
    arrays: dict[str, np.ndarray] = {}
    for name, batch, n, k, g, e in KAT_CASES:
        for key, value in kat_case(batch, n, k, g, e).items():
            arrays[f"{name}/{key}"] = value
    for name, batch, n, k, g, act, asym in RND_CASES:
        for key, value in rnd_case(batch, n, k, g, act, asym).items():
            arrays[f"{name}/{key}"] = value
    out = HERE / "w4a16_golden.npz"
    np.savez_compressed(out, **arrays)
    print(f"wrote {out} ({out.stat().st_size} bytes, {len(arrays)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
