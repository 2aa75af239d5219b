"""CPU tests pinning the oracle (oracle/w4a16_oracle.c) with checks independent of its code:
numpy's own IEEE conversions, float64 brute force, closed forms and invariants. The reference
ships no golden vectors for this path, so these (plus the committed fixtures) are the pins."""

from __future__ import annotations

import math

import numpy as np
import pytest

from fast_kernels.benchmarking.inputs import (
    bf16_bits_to_f32,
    f16_bits_to_f32,
    f32_to_bf16_bits,
    make_case,
    seed_for_case,
)
from oracle import oracle


def test_f32_to_f16_matches_numpy_on_edge_and_random_values() -> None:
    rng = np.random.default_rng(0)
    specials = np.array(
        [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 6.1035156e-05, 6.0e-08,
         5.96e-08, 2.98e-08, 2.99e-08, 1e-12, np.inf, -np.inf, 1.0009765625, 1.00048828125,
         1.00146484375, 2049.0, 2051.0, 3.0517578e-05],
        dtype=np.float32,
    )
    rand = np.concatenate(
        [
            rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
            rng.uniform(-70000, 70000, 5000).astype(np.float32),
            # ties: exact midpoints between neighbouring fp16 values
            (np.arange(1024, 2048, dtype=np.float32) + 0.5),
        ]
    ).astype(np.float32)
    vals = np.concatenate([specials, rand])
    got = oracle.f32_to_f16_bits_array(vals)
    want = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    assert oracle.f32_to_f16_bits(float("nan")) & 0x7C00 == 0x7C00


def test_bf16_round_trip_and_rounding() -> None:
    vals = np.array([1.0, 1.00390625, 1.005859375, 1.0078125, -3.5, 1e-30, 3e38], dtype=np.float32)
    bits = f32_to_bf16_bits(vals)
    # 1.00390625 = 1 + 2^-8 is a tie between 1 and 1+2^-7: rounds to even (1.0)
    assert bits[1] == 0x3F80
    back = bf16_bits_to_f32(bits)
    assert np.all(np.abs(back - vals) <= np.abs(vals) * 2.0**-8)
    lib = oracle.lib()
    for v, b in zip(vals, bits):
        assert lib.fko_f32_to_bf16_bits(float(v)) == b


def test_f32_to_bf16_matches_torch_on_edge_random_and_tie_values() -> None:
    """fko_f32_to_bf16_bits (the oracle's bf16 output rounding) against torch's IEEE round-to-
    nearest-even cast to bfloat16, over the fp16 test's value set plus exact bf16 ties (low 16
    bits 0x8000, both parities of the kept bit), bf16 subnormals, the overflow boundary and
    signed zeros."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    specials = np.array(
        [0.0, -0.0, 1.0, -1.0, 3.3895314e38, 3.3961776e38, 3.4028235e38, 1e-38, 9.18e-41,
         -9.18e-41, 1.0e-45, np.inf, -np.inf, 1.00390625, 1.01171875, 65504.0, 1e9, -1e9],
        dtype=np.float32,
    )
    rand = np.concatenate(
        [
            rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
            rng.uniform(-70000, 70000, 5000).astype(np.float32),
        ]
    ).astype(np.float32)
    ties_bits = (rng.integers(0, 2**16, 4000, dtype=np.uint32) << 16) | np.uint32(0x8000)
    ties = ties_bits.view(np.float32)
    ties = ties[np.isfinite(ties)]
    sub_bits = rng.integers(1, 2**23, 1000, dtype=np.uint32) | (
        rng.integers(0, 2, 1000, dtype=np.uint32) << 31)
    vals = np.concatenate([specials, rand, ties, sub_bits.view(np.float32)]).astype(np.float32)
    want = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    lib = oracle.lib()
    got = np.array([lib.fko_f32_to_bf16_bits(float(v)) for v in vals], dtype=np.uint16)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(f32_to_bf16_bits(vals), want)  # the host-side input recipe
    nan = lib.fko_f32_to_bf16_bits(float("nan"))
    assert nan & 0x7F80 == 0x7F80 and nan & 0x7F


def _numpy_dequant(case, group_size):
    q = np.empty((case.n, case.k), dtype=np.float32)
    q[:, 0::2] = case.q_u8 & 0xF
    q[:, 1::2] = case.q_u8 >> 4
    a = np.repeat(f16_bits_to_f32(case.alpha), group_size, axis=1)
    b = np.repeat(f16_bits_to_f32(case.beta), group_size, axis=1)
    return (a * q + b).astype(np.float32)


@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("asym", [False, True])
def test_dequant_bit_exact_vs_numpy(group_size: int, asym: bool) -> None:
    case = make_case(1, 256, 4 * group_size, group_size, asymmetric=asym, seed=3)
    w = oracle.dequant(case.q_u8, case.alpha, case.beta, group_size)
    want = _numpy_dequant(case, group_size).astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(w, want)


def test_dequant_fp32_value_is_exact_for_the_recipe() -> None:
    # alpha*q + beta must be exact in fp32 (so any evaluation order gives the same fp16)
    case = make_case(1, 128, 1024, 128, asymmetric=True, seed=9)
    w32 = _numpy_dequant(case, 128).astype(np.float64)
    q = np.empty((case.n, case.k))
    q[:, 0::2] = case.q_u8 & 0xF
    q[:, 1::2] = case.q_u8 >> 4
    a = np.repeat(f16_bits_to_f32(case.alpha).astype(np.float64), 128, axis=1)
    b = np.repeat(f16_bits_to_f32(case.beta).astype(np.float64), 128, axis=1)
    np.testing.assert_array_equal(w32, a * q + b)


def test_symmetric_code_8_dequantises_to_zero() -> None:
    case = make_case(1, 128, 256, 128)
    case.q_u8[:] = 0x88
    assert np.all(oracle.dequant(case.q_u8, case.alpha, case.beta, 128) == 0)


@pytest.mark.parametrize("group_size", [64, 128])
def test_packets_layout_matches_formula_and_round_trips(group_size: int) -> None:
    n, k = 256, 4 * group_size
    case = make_case(1, n, k, group_size, asymmetric=True, seed=21)
    packets = oracle.pack_packets(case.q_u8, case.alpha, case.beta, group_size)
    ng = k // group_size
    stride = 128 * group_size // 2 + 512
    assert packets.shape == ((n // 128) * ng, stride)
    rng = np.random.default_rng(1)
    for _ in range(500):
        r = int(rng.integers(n))
        col = int(rng.integers(k))
        t, c, g = r // 128, r % 128, col // group_size
        w = (col % group_size) // 8
        row = packets[t * ng + g]
        word = int.from_bytes(row[(w * 128 + c) * 4:(w * 128 + c) * 4 + 4].tobytes(), "little")
        code = (word >> (4 * (col % 8))) & 0xF
        byte = int(case.q_u8[r, col // 2])
        assert code == ((byte >> 4) if col % 2 else (byte & 0xF))
        qb = 128 * group_size // 2
        assert row[qb + 2 * c:qb + 2 * c + 2].view(np.uint16)[0] == case.alpha[r, g]
        assert row[qb + 256 + 2 * c:qb + 258 + 2 * c].view(np.uint16)[0] == case.beta[r, g]
    np.testing.assert_array_equal(
        oracle.dequant_packets(packets, n, k, group_size),
        oracle.dequant(case.q_u8, case.alpha, case.beta, group_size),
    )


def test_group_sums_brute_force() -> None:
    case = make_case(3, 128, 512, 64, seed=4)
    got = oracle.group_sums(case.x, 64)
    want = f16_bits_to_f32(case.x).astype(np.float64).reshape(3, 8, 64).sum(-1)
    np.testing.assert_allclose(got, want, rtol=1e-7, atol=1e-7)


@pytest.mark.parametrize("act", ["f16", "bf16"])
@pytest.mark.parametrize("group_size", [64, 128])
def test_gemv_vs_float64_matmul(act: str, group_size: int) -> None:
    case = make_case(4, 384, 8 * group_size, group_size, act=act, asymmetric=True, seed=17)
    bits, f32 = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size, act)
    w = _numpy_dequant(case, group_size).astype(np.float64)
    want = case.x_f32().astype(np.float64) @ w.T
    np.testing.assert_allclose(f32, want, rtol=1e-6, atol=1e-6)
    round_fn = (lambda v: v.astype(np.float16).view(np.uint16)) if act == "f16" else f32_to_bf16_bits
    np.testing.assert_array_equal(bits, round_fn(f32))


@pytest.mark.parametrize("act", ["f16", "bf16"])
def test_gemv_f32_is_the_float32_sequential_sum(act: str) -> None:
    """The CPU baseline's fp32 accumulation: against numpy summing the same fp32 products in k
    order in float32 (np.cumsum keeps float32 and is sequential), then one cast."""
    case = make_case(2, 128, 1024, 128, act=act, asymmetric=True, seed=23)
    bits = oracle.gemv_f32(case.x, case.q_u8, case.alpha, case.beta, 128, act)
    w = _numpy_dequant(case, 128)  # float32 alpha * q + beta
    prod = case.x_f32()[:, None, :].astype(np.float32) * w[None, :, :].astype(np.float32)
    acc = np.cumsum(prod, axis=2, dtype=np.float32)[:, :, -1]
    round_fn = (lambda v: v.astype(np.float16).view(np.uint16)) if act == "f16" else f32_to_bf16_bits
    np.testing.assert_array_equal(bits, round_fn(acc))


def test_gemv_one_hot_and_identity_scale() -> None:
    case = make_case(1, 128, 256, 64, seed=5)
    case.alpha[:] = np.float16(1.0).view(np.uint16)
    case.beta[:] = 0
    case.x[:] = 0
    case.x[0, 77] = np.float16(1.0).view(np.uint16)
    bits, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 64)
    codes = (case.q_u8[:, 38] >> 4).astype(np.float32)
    np.testing.assert_array_equal(f16_bits_to_f32(bits)[0], codes)


def test_gemv_linearity_and_zero_weights() -> None:
    case = make_case(2, 128, 512, 128, seed=6)
    _, y1 = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    x2 = (f16_bits_to_f32(case.x) * 2).astype(np.float16).view(np.uint16)
    _, y2 = oracle.gemv(x2, case.q_u8, case.alpha, case.beta, 128)
    np.testing.assert_array_equal(y2, 2 * y1)
    case.q_u8[:] = 0x88
    bits, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    assert np.all(bits == 0)


def test_reduce_partials_in_slice_order() -> None:
    p = np.array([[[1e8, 1.0]], [[1.0, 1.0]], [[-1e8, 1.0]]], dtype=np.float32)
    out = f16_bits_to_f32(oracle.reduce_partials(p))
    # fp32 in order: (1e8 + 1) - 1e8 == 0 (the 1 is absorbed), 1+1+1 == 3
    np.testing.assert_array_equal(out, np.array([[0.0, 3.0]], dtype=np.float32))


def test_seed_formula_matches_reference() -> None:
    # decode_linear_w4a16.py:148-149
    assert seed_for_case(1, 4096, 4096, 128) == (1_000_003 + 4096 * 1009 + 4096 * 101 + 128) % (2**31 - 1)
    a = make_case(1, 128, 256, 128)
    b = make_case(1, 128, 256, 128)
    np.testing.assert_array_equal(a.q_u8, b.q_u8)
    np.testing.assert_array_equal(a.x, b.x)


def test_recipe_distributions() -> None:
    case = make_case(1, 1024, 4096, 128, asymmetric=True)
    alpha = f16_bits_to_f32(case.alpha)
    assert alpha.min() >= 0.000999 and alpha.max() <= 0.0201
    codes = np.concatenate([case.q_u8 & 0xF, case.q_u8 >> 4])
    counts = np.bincount(codes.ravel(), minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    beta = f16_bits_to_f32(case.beta)
    want = (-(alpha * case.zero_points.astype(np.float32))).astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(beta, want)
    sym = make_case(1, 128, 256, 128)
    np.testing.assert_array_equal(f16_bits_to_f32(sym.beta), -8 * f16_bits_to_f32(sym.alpha))
    assert math.isclose(float(case.x_f32().std()), 1.0, rel_tol=0.05)
