"""Loader for tests/golden/w4a16_golden.npz (written by tests/golden/make_golden.py)."""

from __future__ import annotations

from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden" / "w4a16_golden.npz"


def load_cases() -> dict[str, dict[str, np.ndarray]]:
    cases: dict[str, dict[str, np.ndarray]] = {}
    with np.load(GOLDEN, allow_pickle=False) as data:
        for key in data.files:
            name, field = key.split("/", 1)
            cases.setdefault(name, {})[field] = data[key]
    return cases


def meta(case: dict[str, np.ndarray]) -> tuple[int, int, int, int, str, bool]:
    batch, n, k, g, act, asym = (int(v) for v in case["meta"])
    return batch, n, k, g, ("bf16" if act else "f16"), bool(asym)
