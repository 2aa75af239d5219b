"""GPU tests of the native packet formats (symmetric: no beta; asymmetric: int4 zero points).

Pins:
  * layout: a native packet is the oracle's reference packet (oracle.pack_packets) with its 256
    beta bytes dropped (symmetric) or replaced by the 128 zero points, two per byte, low nibble
    for the even column (asymmetric);
  * conversions: reference -> native -> reference reproduces oracle.pack_packets byte for byte;
    reference packets whose betas are not half_rn(-alpha * zp) are rejected;
  * forward: over native packets the output equals, bit for bit, the same launch over the
    reference packets, and is within the GEMV bar of the oracle (rel 1e-2,
    abs 1e-2 * sqrt(K) * max|alpha|).
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import gpu_available

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="needs a GPU"),
]

torch = pytest.importorskip("torch")

from fast_kernels.benchmarking.inputs import make_case  # noqa: E402
from fast_kernels.ops import (  # noqa: E402
    arc_w4a16_forward,
    arc_w4a16_forward_native,
    arc_w4a16_plan,
    convert_arc_to_native_packets,
    convert_native_to_arc_packets,
    pack_arc_w4a16_packets,
    pack_native_w4a16_packets,
    packet_stride_bytes,
)
from oracle import oracle  # noqa: E402
from test_gpu_w4a16_parity import _assert_gemv_close, _bits, _upload  # noqa: E402

DEV = "cuda"


def _fmt(asym: bool) -> str:
    return "native_asym" if asym else "native_sym"


def _expected_native(case, asym: bool) -> np.ndarray:
    ref = oracle.pack_packets(case.q_u8, case.alpha, case.beta, case.group_size)
    head = 64 * case.group_size + 256  # code words and alpha
    if not asym:
        return np.ascontiguousarray(ref[:, :head])
    ng = case.k // case.group_size
    # zero points in packet order: packet (tile t, group g), column c -> zp[t*128 + c, g]
    zp = case.zero_points.reshape(case.n // 128, 128, ng).transpose(0, 2, 1).reshape(-1, 128)
    nibbles = (zp[:, 0::2] | (zp[:, 1::2] << 4)).astype(np.uint8)
    return np.ascontiguousarray(np.concatenate([ref[:, :head], nibbles], axis=1))


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("shape", [(128, 256), (512, 2048)])
def test_pack_native_layout(asym: bool, group_size: int, shape: tuple[int, int]) -> None:
    n, k = shape
    case = make_case(1, n, k, group_size, asymmetric=asym, seed=31 + n + group_size)
    _, q, a, _ = _upload(case)
    zp = torch.from_numpy(case.zero_points).to(DEV) if asym else None
    packets = pack_native_w4a16_packets(q, a, zp, group_size=group_size, packet_format=_fmt(asym))
    assert packets.shape[1] == packet_stride_bytes(group_size, _fmt(asym))
    np.testing.assert_array_equal(packets.cpu().numpy(), _expected_native(case, asym))


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("recipe", ["baseline", "reference"])
def test_arc_native_round_trip(asym: bool, group_size: int, recipe: str) -> None:
    n, k = 384, 8 * group_size
    if recipe == "reference" and not asym:
        pytest.skip("the reference recipe always draws zero points")
    case = make_case(1, n, k, group_size, asymmetric=asym, seed=7 + group_size, recipe=recipe)
    arc = torch.from_numpy(oracle.pack_packets(case.q_u8, case.alpha, case.beta, group_size)).to(DEV)
    native = convert_arc_to_native_packets(arc, n=n, k=k, group_size=group_size,
                                           packet_format=_fmt(asym))
    np.testing.assert_array_equal(native.cpu().numpy(), _expected_native(case, asym))
    back = convert_native_to_arc_packets(native, n=n, k=k, group_size=group_size,
                                         packet_format=_fmt(asym))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(back.cpu().numpy(), arc.cpu().numpy())


def test_arc_to_native_rejects_other_betas() -> None:
    case = make_case(1, 256, 1024, 128, asymmetric=True, seed=3)
    arc_np = oracle.pack_packets(case.q_u8, case.alpha, case.beta, 128)
    arc = torch.from_numpy(arc_np).to(DEV)
    # zero points other than 8: not symmetric
    with pytest.raises(ValueError, match="symmetric"):
        convert_arc_to_native_packets(arc, n=256, k=1024, group_size=128, packet_format="native_sym")
    # one beta nudged by one ulp: no integer zero point reproduces it
    bad = arc_np.copy()
    off = 64 * 128 + 256 + 2 * 77  # beta of column 77 in the first packet
    bits = int(bad[0, off]) | (int(bad[0, off + 1]) << 8)
    bits ^= 1
    bad[0, off], bad[0, off + 1] = bits & 0xFF, bits >> 8
    with pytest.raises(ValueError, match="affine"):
        convert_arc_to_native_packets(torch.from_numpy(bad).to(DEV), n=256, k=1024, group_size=128,
                                      packet_format="native_asym")
    # the flag is cleared per call: a good conversion afterwards succeeds
    convert_arc_to_native_packets(arc, n=256, k=1024, group_size=128, packet_format="native_asym")


def _forward_pair(case, asym: bool, **kwargs) -> tuple[np.ndarray, np.ndarray]:
    x, q, a, b = _upload(case)
    g = case.group_size
    arc = pack_arc_w4a16_packets(q, a, b, group_size=g)
    native = convert_arc_to_native_packets(arc, n=case.n, k=case.k, group_size=g,
                                           packet_format=_fmt(asym))
    y_arc = arc_w4a16_forward(x, arc, n=case.n, k=case.k, group_size=g, impl="scalar", **kwargs)
    y_nat = arc_w4a16_forward_native(x, native, n=case.n, k=case.k, group_size=g,
                                     packet_format=_fmt(asym), **kwargs)
    torch.cuda.synchronize()
    return _bits(y_nat), _bits(y_arc)


@pytest.mark.parametrize("asym", [False, True])
@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("act", ["f16", "bf16"])
def test_forward_native_matches_reference_packets(asym, group_size, batch, act) -> None:
    case = make_case(batch, 512, 16 * group_size, group_size, act=act, asymmetric=asym,
                     seed=1000 + batch + group_size)
    y_nat, y_arc = _forward_pair(case, asym)
    np.testing.assert_array_equal(y_nat, y_arc)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size, act)
    _assert_gemv_close(y_nat, ref, case, f"{_fmt(asym)} {act} G={group_size} M={batch}")


@pytest.mark.parametrize(
    "shape,act,asym",
    [
        ((1, 1024, 2048, 128), "f16", False),    # 32-column slices
        ((1, 10240, 4096, 128), "f16", True),    # 64-column slices
        ((1, 4096, 14336, 128), "bf16", False),  # narrow slices + K split (fix-up)
        ((1, 8192, 8192, 128), "f16", False),    # Llama-70B o, whole tiles + K split
        ((2, 4096, 4096, 64), "f16", True),      # two rows, K runs per tile
        ((16, 4096, 4096, 64), "bf16", True),    # matrix-core tile
    ],
)
def test_forward_native_plans_match_oracle(shape, act, asym) -> None:
    batch, n, k, g = shape
    plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=g,
                          activation_dtype=torch.float16 if act == "f16" else torch.bfloat16)
    case = make_case(batch, n, k, g, act=act, asymmetric=asym)
    y_nat, y_arc = _forward_pair(case, asym)
    np.testing.assert_array_equal(y_nat, y_arc)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, g, act)
    _assert_gemv_close(y_nat, ref, case, f"{shape} {act} plan={plan}")


@pytest.mark.parametrize("split", [3, 7])
def test_forward_native_forced_split(split: int) -> None:
    case = make_case(1, 1024, 64 * 128, 128, asymmetric=True, seed=99)
    y_nat, y_arc = _forward_pair(case, True, split_k_slices=1)
    np.testing.assert_array_equal(y_nat, y_arc)
    x, q, a, b = _upload(case)
    arc = pack_arc_w4a16_packets(q, a, b, group_size=128)
    native = convert_arc_to_native_packets(arc, n=1024, k=64 * 128, group_size=128,
                                           packet_format="native_asym")
    # the native forward with a Stream-K run length the automatic plan would not pick
    y = arc_w4a16_forward_native(x, native, n=1024, k=64 * 128, group_size=128,
                                 packet_format="native_asym", split_k_slices=split)
    torch.cuda.synchronize()
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    _assert_gemv_close(_bits(y), ref, case, f"native split={split}")
