"""GPU tests of the native packet formats (symmetric: no beta; asymmetric: int4 zero points).

Pins:
  * layout: native slabs are the oracle's reference packets (oracle.pack_packets) cut into
    32-column slices, ordered [tile][slice][group], code words in quarter order, alphas in column
    pairs, betas dropped (symmetric) or replaced by the slice's 32 zero points (asymmetric);
  * conversions: reference -> native -> reference reproduces oracle.pack_packets byte for byte;
    reference packets whose betas are not half_rn(-alpha * zp) are rejected;
  * forward: over native slabs the output is within the GEMV bar of the oracle (rel 1e-2,
    abs 1e-2 * sqrt(K) * max|alpha|), like the forward over the reference packets the slabs came
    from (the two launches differ in slice width and K split, so in fp32 summation order only).
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


def _native_word_offset(g: int, i: int, t: int, n: int, j: int) -> int:
    """Byte offset in a slab of word j of the unit (column 16 i + n, quarter t)."""
    return i * 1024 + (16 * t + n) * 16 + 4 * j if g == 128 else (16 * t + n) * 16 + i * 8 + 4 * j


def _expected_native(case, asym: bool) -> np.ndarray:
    """Native slabs rearranged from the oracle's reference packets. Slab (tile, slice, group):
    the slice's code words in quarter order (column 16 i + n has G/8 words in four quarters of
    U = G/32; lane 16 t + n of a wave owns quarter t of columns n and n + 16), then 16 records,
    one per column pair: (alpha[n], alpha[n + 16]) and, asymmetric, (-zp[n], -zp[n + 16]) as
    fp16 (zp = 0 as -0)."""
    g = case.group_size
    ng = case.k // g
    tiles = case.n // 128
    u = g // 32
    ref = oracle.pack_packets(case.q_u8, case.alpha, case.beta, g).reshape(tiles, ng, -1)
    words = ref[:, :, : 64 * g].copy().view(np.uint32).reshape(tiles, ng, g // 8, 128)
    alpha = ref[:, :, 64 * g : 64 * g + 256].copy().view(np.uint16).reshape(tiles, ng, 128)
    rec = 8 if asym else 4
    stride = 16 * g + 16 * rec
    out = np.zeros((tiles, 4, ng, stride), dtype=np.uint8)
    codes = np.zeros((tiles, 4, ng, 4 * g), dtype=np.uint32)  # 16 g bytes per slab
    for i in range(2):
        for t in range(4):
            for n in range(16):
                for j in range(u):
                    dst = _native_word_offset(g, i, t, n, j) // 4
                    col = np.arange(4) * 32 + 16 * i + n  # this column in each of the 4 slices
                    codes[:, :, :, dst] = words[:, :, t * u + j, col].transpose(0, 2, 1)
    out[..., : 16 * g] = codes.view(np.uint8).reshape(tiles, 4, ng, 16 * g)
    records = np.zeros((tiles, 4, ng, 16, rec), dtype=np.uint8)
    for i in range(2):
        col = np.arange(4)[:, None] * 32 + 16 * i + np.arange(16)[None, :]  # [slice, n]
        a = alpha[:, :, col].transpose(0, 2, 1, 3)  # [t, s, g, n]
        records[..., 2 * i] = (a & 0xFF).astype(np.uint8)
        records[..., 2 * i + 1] = (a >> 8).astype(np.uint8)
    if asym:
        zp = case.zero_points.reshape(tiles, 4, 32, ng).transpose(0, 1, 3, 2)  # [t, s, g, col]
        for i in range(2):
            neg = (-zp[..., 16 * i : 16 * i + 16].astype(np.float16)).view(np.uint16)
            neg = np.where(zp[..., 16 * i : 16 * i + 16] == 0, np.uint16(0x8000), neg)
            records[..., 4 + 2 * i] = (neg & 0xFF).astype(np.uint8)
            records[..., 5 + 2 * i] = (neg >> 8).astype(np.uint8)
    out[..., 16 * g :] = records.reshape(tiles, 4, ng, 16 * rec)
    return out.reshape(tiles * 4 * ng, stride)


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
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 7, 8, 16, 33])
@pytest.mark.parametrize("act", ["f16", "bf16"])
def test_forward_native_matches_reference_packets(asym, group_size, batch, act) -> None:
    case = make_case(batch, 512, 16 * group_size, group_size, act=act, asymmetric=asym,
                     seed=1000 + batch + group_size)
    y_nat, y_arc = _forward_pair(case, asym)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size, act)
    _assert_gemv_close(y_nat, ref, case, f"{_fmt(asym)} {act} G={group_size} M={batch}")
    _assert_gemv_close(y_arc, ref, case, f"arc {act} G={group_size} M={batch}")


@pytest.mark.parametrize(
    "shape,act,asym,cols",
    [
        ((1, 1024, 2048, 128), "f16", False, 16),    # 32 slices, a half slice per workgroup
        ((1, 10240, 4096, 128), "f16", True, 64),    # 320 slices in 160 slice pairs
        ((1, 4096, 14336, 128), "bf16", False, 16),  # 128 slices, a half slice per workgroup
        ((1, 57344, 8192, 128), "bf16", False, 32),  # Llama-70B gate_up, eight slices on 224 CUs
        ((1, 8192, 28672, 128), "bf16", False, 32),  # Llama-70B down: long K, runs of 112 (fix-up)
        ((1, 12288, 1024, 64), "f16", False, 64),    # slice pairs over 16 groups
        ((1, 28672, 4096, 128), "bf16", True, 32),   # Llama-8B gate_up: 4 slices per CU on 224 CUs
        ((1, 12288, 37 * 64, 64), "bf16", True, 64),  # slice pairs, odd group count
        ((1, 10240, 7 * 128, 128), "f16", False, 64),  # slice pairs, odd group count at G=128
        ((1, 12288, 130 * 64, 64), "f16", False, 32),  # pairs would fit, but K is long
        ((3, 1024, 37 * 64, 64), "f16", True, 32),   # odd group count over two 32-group chunks
        ((2, 2048, 130 * 64, 64), "bf16", False, 32),  # three 64-group chunks, the last of 2 groups
        ((2, 4096, 4096, 64), "f16", True, 32),      # two rows
        ((8, 4096, 4096, 64), "bf16", True, 32),     # eight rows: matrix cores, stream schedule
        ((16, 4096, 4096, 64), "bf16", True, 32),    # sixteen rows: matrix-core stream, 128 slices
        ((16, 4096, 8192, 64), "bf16", True, 32),    # long K: matrix-core stream, K in 2 parts
        ((16, 4096, 32768, 128), "f16", False, 32),   # K in 8 parts of 32 groups
        ((5, 4096, 8192, 64), "f16", False, 32),     # staging past the registers: dot2 runs
    ],
)
def test_forward_native_plans_match_oracle(shape, act, asym, cols) -> None:
    batch, n, k, g = shape
    plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=g,
                          activation_dtype=torch.float16 if act == "f16" else torch.bfloat16,
                          packet_format=2 if asym else 1)
    assert plan["slice_cols"] == cols, plan
    case = make_case(batch, n, k, g, act=act, asymmetric=asym)
    y_nat, _ = _forward_pair(case, asym)
    if n > 8192:  # the oracle checks a spread subset of rows of the large shape
        rows = np.unique(np.linspace(0, n - 1, 512).astype(int))
        ref, _ = oracle.gemv(case.x, np.ascontiguousarray(case.q_u8[rows]),
                             np.ascontiguousarray(case.alpha[rows]),
                             np.ascontiguousarray(case.beta[rows]), g, act)
        _assert_gemv_close(y_nat[:, rows], ref, case, f"{shape} {act} plan={plan}")
        return
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, g, act)
    _assert_gemv_close(y_nat, ref, case, f"{shape} {act} plan={plan}")


@pytest.mark.parametrize("split", [1, 3, 7])
def test_forward_native_forced_split(split: int) -> None:
    """Forced K runs of ceil(64/split) groups over 32-column slices; 3 and 7 give runs that
    straddle slices, so a slice is finished from the partials of up to 3 workgroups."""
    case = make_case(1, 1024, 64 * 128, 128, asymmetric=True, seed=99)
    x, q, a, b = _upload(case)
    arc = pack_arc_w4a16_packets(q, a, b, group_size=128)
    native = convert_arc_to_native_packets(arc, n=1024, k=64 * 128, group_size=128,
                                           packet_format="native_asym")
    plan = arc_w4a16_plan(batch=1, n=1024, k=64 * 128, group_size=128, split_k_slices=split,
                          packet_format=2)
    assert plan["groups_per_workgroup"] == -(-64 // split) and plan["slice_cols"] == 32
    y = arc_w4a16_forward_native(x, native, n=1024, k=64 * 128, group_size=128,
                                 packet_format="native_asym", split_k_slices=split)
    torch.cuda.synchronize()
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    _assert_gemv_close(_bits(y), ref, case, f"native split={split}")


def test_forward_native_deterministic() -> None:
    case = make_case(1, 4096, 14336, 128, seed=5)  # K split in two: the fix-up path
    x, q, a, b = _upload(case)
    native = convert_arc_to_native_packets(pack_arc_w4a16_packets(q, a, b, group_size=128),
                                           n=4096, k=14336, group_size=128)
    ys = [_bits(arc_w4a16_forward_native(x, native, n=4096, k=14336, group_size=128))
          for _ in range(3)]
    for y in ys[1:]:
        np.testing.assert_array_equal(y, ys[0])
