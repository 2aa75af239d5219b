"""The CPU oracle against the committed golden vectors (tests/golden/w4a16_golden.npz).

The kat_* cases hold answers computed with exact integer arithmetic, independent of the oracle,
so the oracle must reproduce them bit-for-bit (dequant and y). The rnd_* cases freeze the
oracle's own outputs on seeded inputs; a change in the oracle or the input recipe fails here.
"""

from __future__ import annotations

import hashlib

import numpy as np
import pytest

from golden_vectors import load_cases, meta

from fast_kernels.benchmarking.inputs import make_case
from oracle import oracle

CASES = load_cases()
KAT = sorted(k for k in CASES if k.startswith("kat_"))
RND = sorted(k for k in CASES if k.startswith("rnd_"))


def _sha(a: np.ndarray) -> bytes:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).digest()


def test_golden_file_has_both_kinds() -> None:
    assert len(KAT) >= 2 and len(RND) >= 4


@pytest.mark.parametrize("name", KAT)
def test_oracle_reproduces_known_answers(name: str) -> None:
    c = CASES[name]
    batch, n, k, g, act, _ = meta(c)
    np.testing.assert_array_equal(oracle.dequant(c["q_u8"], c["alpha"], c["beta"], g), c["dequant"])
    y, y32 = oracle.gemv(c["x"], c["q_u8"], c["alpha"], c["beta"], g, act)
    np.testing.assert_array_equal(y, c["y"])
    np.testing.assert_array_equal(y32.astype(np.float16).view(np.uint16), c["y"])
    packets = oracle.pack_packets(c["q_u8"], c["alpha"], c["beta"], g)
    np.testing.assert_array_equal(oracle.dequant_packets(packets, n, k, g), c["dequant"])


@pytest.mark.parametrize("name", RND)
def test_recipe_regenerates_golden_inputs(name: str) -> None:
    c = CASES[name]
    batch, n, k, g, act, asym = meta(c)
    case = make_case(batch, n, k, g, act=act, asymmetric=asym)
    for field in ("x", "q_u8", "alpha", "beta"):
        np.testing.assert_array_equal(getattr(case, field), c[field], err_msg=field)


@pytest.mark.parametrize("name", RND)
def test_oracle_matches_frozen_outputs(name: str) -> None:
    c = CASES[name]
    batch, n, k, g, act, _ = meta(c)
    w = oracle.dequant(c["q_u8"], c["alpha"], c["beta"], g)
    assert _sha(w) == c["dequant_sha256"].tobytes()
    np.testing.assert_array_equal(w[0], c["dequant_row0"])
    packets = oracle.pack_packets(c["q_u8"], c["alpha"], c["beta"], g)
    assert _sha(packets) == c["packets_sha256"].tobytes()
    np.testing.assert_array_equal(oracle.group_sums(c["x"], g, act), c["group_sums"])
    y, y32 = oracle.gemv(c["x"], c["q_u8"], c["alpha"], c["beta"], g, act)
    np.testing.assert_array_equal(y, c["y"])
    np.testing.assert_array_equal(y32, c["y_f32"])
