"""GPU parity tests: the HIP library (through fast_kernels._native -> the C ABI) against the CPU
oracle on identical seeded inputs.

Bars: dequantisation and packing are bit-exact; GEMV outputs must satisfy
|y - y_ref| <= atol + rtol*|y_ref| with rtol = 1e-2 and atol = 1e-2*sqrt(K)*max|alpha| (the
benchmark configuration's tolerance for fp32 accumulation), where y_ref is the oracle's
double-accumulated result rounded once to the output dtype. The reference's own tests use
atol = rtol = 1e-2 (tests/gpu/test_decode_quant_linear.py:102); the suite gate is atol 0.0625,
rtol 0.01 (benchmarks/suites/decode_linear_w4a16.toml:21-23).
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import gpu_available

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="needs a GPU"),
]

torch = pytest.importorskip("torch")

from fast_kernels.benchmarking.inputs import bf16_bits_to_f32, f16_bits_to_f32, make_case  # noqa: E402
from fast_kernels.ops import (  # noqa: E402
    arc_packet_stride_bytes,
    arc_w4a16_forward,
    arc_w4a16_plan,
    compute_arc_w4a16_group_sums,
    cublaslt_fp16_after_dequant,
    dequant_arc_w4a16_packets_to_fp16,
    dequant_w4a16_to_fp16,
    pack_arc_w4a16_packets,
)
from oracle import oracle  # noqa: E402
from fast_kernels.native import native_module  # noqa: E402
from fast_kernels.ops.decode_quant_linear import _IMPL_KERNEL  # noqa: E402

DEV = "cuda"


def _dev_bits(a: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).view(dtype).to(DEV)


def _upload(case):
    act_dtype = torch.float16 if case.act == "f16" else torch.bfloat16
    x = _dev_bits(case.x.view(np.int16), torch.int16).view(act_dtype)
    q = torch.from_numpy(case.q_u8).to(DEV)
    a = _dev_bits(case.alpha.view(np.int16), torch.int16).view(torch.float16)
    b = _dev_bits(case.beta.view(np.int16), torch.int16).view(torch.float16)
    return x, q, a, b


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _to_f32(bits: np.ndarray, act: str) -> np.ndarray:
    return f16_bits_to_f32(bits) if act == "f16" else bf16_bits_to_f32(bits)


def _assert_gemv_close(y_bits: np.ndarray, ref_bits: np.ndarray, case, label: str) -> None:
    y = _to_f32(y_bits, case.act).astype(np.float64)
    ref = _to_f32(ref_bits, case.act).astype(np.float64)
    max_alpha = float(f16_bits_to_f32(case.alpha).max())
    atol = 1e-2 * math.sqrt(case.k) * max_alpha
    rtol = 1e-2
    assert np.all(np.isfinite(y)), f"{label}: non-finite outputs"
    err = np.abs(y - ref)
    bound = atol + rtol * np.abs(ref)
    worst = int(np.argmax(err - bound))
    assert np.all(err <= bound), (
        f"{label}: max |err| {err.max():.4g} (bound {bound.flat[worst]:.4g} at {worst}), "
        f"atol={atol:.4g}"
    )


@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("shape", [(128, 256), (384, 1024), (4096, 4096)])
def test_dequant_bit_exact(group_size: int, shape: tuple[int, int]) -> None:
    n, k = shape
    case = make_case(1, n, k, group_size, asymmetric=True, seed=11 + n + k + group_size)
    _, q, a, b = _upload(case)
    w = dequant_w4a16_to_fp16(q, a, b, group_size=group_size)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(w), oracle.dequant(case.q_u8, case.alpha, case.beta, group_size))


@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("shape", [(128, 256), (512, 2048)])
def test_packets_byte_exact_and_round_trip(group_size: int, shape: tuple[int, int]) -> None:
    n, k = shape
    case = make_case(1, n, k, group_size, asymmetric=True, seed=5 + n + group_size)
    _, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=group_size)
    assert tuple(packets.shape) == ((n // 128) * (k // group_size), arc_packet_stride_bytes(group_size))
    ref_packets = oracle.pack_packets(case.q_u8, case.alpha, case.beta, group_size)
    np.testing.assert_array_equal(packets.cpu().numpy(), ref_packets)
    w = dequant_arc_w4a16_packets_to_fp16(packets, n=n, k=k, group_size=group_size)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(w), oracle.dequant(case.q_u8, case.alpha, case.beta, group_size))


@pytest.mark.parametrize("group_size", [64, 128])
def test_group_sums_match_oracle(group_size: int) -> None:
    case = make_case(5, 128, 8 * group_size, group_size, seed=77)
    x, _, _, _ = _upload(case)
    sums = compute_arc_w4a16_group_sums(x, group_size=group_size)
    ref = oracle.group_sums(case.x, group_size)
    np.testing.assert_allclose(sums.cpu().numpy(), ref, rtol=1e-6, atol=1e-5)


def _run_forward(case, **kwargs) -> np.ndarray:
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=case.group_size)
    y = arc_w4a16_forward(x, packets, n=case.n, k=case.k, group_size=case.group_size, **kwargs)
    torch.cuda.synchronize()
    return _bits(y)


@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 7, 8, 12, 16, 33])
@pytest.mark.parametrize("asym", [False, True])
def test_forward_small_matches_oracle(group_size: int, batch: int, asym: bool) -> None:
    case = make_case(batch, 256, 8 * group_size, group_size, asymmetric=asym)
    y = _run_forward(case)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size)
    _assert_gemv_close(y, ref, case, f"G={group_size} M={batch}")


@pytest.mark.parametrize(
    "shape",
    [
        (1, 4096, 4096, 128),    # config 0 / Llama-7B o
        (1, 12288, 4096, 128),   # Llama-7B qkv
        (1, 22016, 4096, 128),   # Llama-7B gate_up
        (1, 4096, 11008, 128),   # Llama-7B down
        (1, 8192, 8192, 128),    # Llama-70B o
        (1, 10240, 8192, 128),   # Llama-70B qkv
    ],
)
def test_forward_baseline_shapes_match_oracle(shape: tuple[int, int, int, int]) -> None:
    batch, n, k, g = shape
    case = make_case(batch, n, k, g)
    y = _run_forward(case)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, g)
    _assert_gemv_close(y, ref, case, f"{shape}")


@pytest.mark.parametrize(
    "shape,act,asym,want",
    [
        # (batch, n, k, G), activation, asymmetric, (slice_cols, groups per workgroup) on 256 CUs
        ((1, 1024, 2048, 128), "f16", False, (16, 16)),    # 8 tiles -> 64 16-column eighths
        ((1, 10240, 4096, 128), "f16", True, (64, 32)),    # 80 tiles -> 160 64-column slices
        ((1, 4096, 14336, 128), "bf16", False, (32, 56)),  # narrow slices + K split (fix-up)
        ((2, 4096, 4096, 64), "f16", True, (32, 64)),      # two rows: matrix-core stream kernel
        ((2, 1024, 8192, 64), "bf16", True, (128, 8)),     # two rows, 16 runs per tile
        ((3, 1024, 37 * 64, 64), "f16", True, (128, 19)),  # odd group count, runs of 19 and 18
        ((2, 2048, 130 * 64, 64), "bf16", False, (128, 9)),  # 130 groups, runs of 9 across chunks
        ((5, 1024, 4096, 128), "bf16", False, (32, 32)),   # five rows: matrix-core stream kernel,
                                                           # one packet quarter per workgroup
    ],
)
def test_forward_column_slices_match_oracle(shape, act, asym, want) -> None:
    """The automatic plan's 64-, 32- and 16-column slices, alone and with K split across
    workgroups, its K splits for several rows, and the matrix-core stream kernel at five."""
    batch, n, k, g = shape
    plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=g,
                          activation_dtype=torch.float16 if act == "f16" else torch.bfloat16)
    if torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert (plan["slice_cols"], plan["groups_per_workgroup"]) == want
    case = make_case(batch, n, k, g, act=act, asymmetric=asym)
    y = _run_forward(case)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, g, act)
    _assert_gemv_close(y, ref, case, f"{shape} {act} plan={plan}")


@pytest.mark.parametrize("act", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(1, 57344, 8192, 128), (1, 8192, 28672, 128)])
def test_forward_llama70b_large_rows_subset(act: str, shape: tuple[int, int, int, int]) -> None:
    """Full-size gate_up / down GEMV; the oracle checks a spread subset of 768 output rows."""
    batch, n, k, g = shape
    case = make_case(batch, n, k, g, act=act)
    y = _run_forward(case)
    rows = np.unique(np.concatenate([np.arange(256), np.linspace(256, n - 257, 256).astype(int), np.arange(n - 256, n)]))
    ref, _ = oracle.gemv(
        case.x,
        np.ascontiguousarray(case.q_u8[rows]),
        np.ascontiguousarray(case.alpha[rows]),
        np.ascontiguousarray(case.beta[rows]),
        g,
        act,
    )
    _assert_gemv_close(y[:, rows], ref, case, f"{shape} {act}")


@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("batch", [1, 2, 4, 8, 16])
def test_forward_bf16_matches_oracle(group_size: int, batch: int) -> None:
    case = make_case(batch, 1024, 16 * group_size, group_size, act="bf16")
    y = _run_forward(case)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size, "bf16")
    _assert_gemv_close(y, ref, case, f"bf16 G={group_size} M={batch}")


@pytest.mark.parametrize("split", [1, 2, 3, 5, 7, 16, 64])
def test_forced_split_k_fixup_matches_oracle(split: int) -> None:
    """Stream-K runs of ceil(64/split) groups; 3, 5 and 7 give runs that straddle tiles, so a
    tile is finished from partials of up to 3 workgroups."""
    case = make_case(1, 1024, 64 * 128, 128, seed=99)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=128)
    from fast_kernels.native import native_module
    from fast_kernels.ops import arc_workspace

    native = native_module()
    plan = arc_w4a16_plan(batch=1, n=1024, k=64 * 128, group_size=128, split_k_slices=split)
    assert plan["groups_per_workgroup"] == -(-64 // split)
    ws = arc_workspace(x.device, max(1, plan["workspace_bytes"]))
    out = torch.empty((1, 1024), device=DEV, dtype=torch.float16)
    stream = torch.cuda.current_stream().cuda_stream
    native.arc_w4a16_forward_ex(
        x.data_ptr(), packets.data_ptr(), out.data_ptr(), ws.data_ptr(), ws.numel(),
        1, 1024, 64 * 128, 128, arc_packet_stride_bytes(128), 0, split, stream,
    )
    torch.cuda.synchronize()
    y = _bits(out)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    _assert_gemv_close(y, ref, case, f"split={split}")


def test_reference_split_k_protocol_with_partials() -> None:
    """Reference test_arc_split_k_override_matches_explicit_reference (:171-207): 4 slices and a
    caller partials buffer; also the partials must sum to the direct result."""
    case = make_case(8, 128, 4 * 128, 128, asymmetric=True, seed=4242)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=128)
    partials = torch.empty((4, 8, 128), device=DEV, dtype=torch.float32)
    y = arc_w4a16_forward(x, packets, n=128, k=512, group_size=128, split_k_slices=4, partials=partials)
    torch.cuda.synchronize()
    ref, ref32 = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    _assert_gemv_close(_bits(y), ref, case, "split-K protocol")
    np.testing.assert_array_equal(_bits(y), oracle.reduce_partials(partials.cpu().numpy()))
    np.testing.assert_allclose(partials.sum(0).cpu().numpy(), ref32, rtol=1e-4, atol=1e-3)


def test_split_k_more_slices_than_needed_writes_zero_partials() -> None:
    # NG = 4, S = 3 -> ceil(4/3) = 2 groups per slice: slice 2 is empty and must contribute 0.
    case = make_case(1, 128, 4 * 64, 64, seed=3)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=64)
    partials = torch.full((3, 1, 128), float("nan"), device=DEV, dtype=torch.float32)
    y = arc_w4a16_forward(x, packets, n=128, k=256, group_size=64, split_k_slices=3, partials=partials)
    torch.cuda.synchronize()
    assert torch.all(partials[2] == 0)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 64)
    _assert_gemv_close(_bits(y), ref, case, "empty slice")


def test_forward_is_deterministic_across_calls() -> None:
    case = make_case(1, 4096, 4096, 128)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=128)
    outs = [_bits(arc_w4a16_forward(x, packets, n=4096, k=4096, group_size=128)) for _ in range(5)]
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])


def test_special_case_zero_weights_give_zero() -> None:
    # symmetric zp = 8 and every code 8 => every weight is exactly 0 => the explicit formula gives
    # y == 0. The GEMV folds the nibble-unpack bias into per-group activation sums
    # (sum((1024+q)x) - 1024*sum(x)), as the reference kernel folds beta * sum(x)
    # (arc_w4a16.cu:276-294), so the cancellation leaves fp32 rounding residue instead of an exact
    # zero. A worst-case fp32 bound of that residue (about 2^-19 * 1032 * sum_g alpha_g *
    # sum_{k in g} |x_k|) is not tighter than the GEMV tolerance itself, so the test holds it to
    # 1e-4, 45 times below atol = 1e-2*sqrt(K)*max|alpha| ~ 4.5e-3 at this shape.
    case = make_case(2, 256, 512, 128)
    case.q_u8[:] = 0x88
    y = np.abs(f16_bits_to_f32(_run_forward(case)))
    assert y.max() < 1e-4, y.max()


def test_special_case_one_hot_recovers_codes() -> None:
    # alpha = 1, beta = 0, x = e_j  =>  y[n] = q[n, j] exactly
    n, k, g = 256, 256, 64
    case = make_case(1, n, k, g, seed=8)
    case.alpha[:] = np.float16(1.0).view(np.uint16)
    case.beta[:] = 0
    j = 37
    case.x[:] = 0
    case.x[0, j] = np.float16(1.0).view(np.uint16)
    y = f16_bits_to_f32(_run_forward(case))
    codes = (case.q_u8[:, j // 2] >> (4 * (j % 2))) & 0xF
    np.testing.assert_array_equal(y[0], codes.astype(np.float32))


def test_identical_rows_give_identical_outputs() -> None:
    case = make_case(4, 512, 1024, 128)
    case.x[1:] = case.x[0]
    y = _run_forward(case)
    for m in range(1, 4):
        np.testing.assert_array_equal(y[m], y[0])


def test_linearity_in_activations() -> None:
    # y(2x) == 2 y(x) exactly up to the final rounding (scaling by 2 is exact in fp16/fp32)
    case = make_case(1, 1024, 4096, 128)
    y1 = f16_bits_to_f32(_run_forward(case))
    x2 = (f16_bits_to_f32(case.x) * 2).astype(np.float16).view(np.uint16)
    case.x[:] = x2
    y2 = f16_bits_to_f32(_run_forward(case))
    np.testing.assert_array_equal(y2, 2 * y1)


def test_vendor_baseline_matches_oracle() -> None:
    case = make_case(4, 1024, 2048, 128)
    x, q, a, b = _upload(case)
    y = cublaslt_fp16_after_dequant(x, q, a, b, group_size=128)
    torch.cuda.synchronize()
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    _assert_gemv_close(_bits(y), ref, case, "hipBLASLt")


def test_tc_impl_and_env_override(monkeypatch: pytest.MonkeyPatch) -> None:
    """Reference test_arc_impl_env_override_matches_explicit_reference (:210-245)."""
    case = make_case(4, 128, 512, 128, seed=5150)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    _assert_gemv_close(_run_forward(case, impl="tc"), ref, case, "impl=tc")
    monkeypatch.setenv("FK_ARC_W4A16_IMPL", "tc")
    _assert_gemv_close(_run_forward(case), ref, case, "env impl=tc")
    monkeypatch.setenv("FK_ARC_W4A16_IMPL", "scalar")
    _assert_gemv_close(_run_forward(case), ref, case, "env impl=scalar")


@pytest.mark.parametrize("impl,batch", [("scalar", 8), ("scalar", 16), ("scalar", 33),
                                        ("mfma", 1), ("mfma", 2), ("mfma", 5), ("mfma", 33)])
@pytest.mark.parametrize("asym", [False, True])
def test_forced_kernel_impls_match_oracle(impl: str, batch: int, asym: bool) -> None:
    """impl "scalar" keeps every batch on the dot2 loop and "mfma" on the matrix-core kernel:
    both within the GEMV bar of the oracle at the batch sizes the automatic dispatch sends to the
    other kernel."""
    case = make_case(batch, 512, 16 * 64, 64, asymmetric=asym, seed=4000 + batch)
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 64)
    _assert_gemv_close(_run_forward(case, impl=impl), ref, case, f"impl={impl} M={batch}")
    want = 16 if impl == "mfma" else min(8, 1 << (batch - 1).bit_length())
    plan = arc_w4a16_plan(batch=batch, n=512, k=1024, group_size=64, kernel=_IMPL_KERNEL[impl])
    assert plan["m_tile"] == want


@pytest.mark.parametrize("kernel", [1, 2])
@pytest.mark.parametrize("batch", [3, 8])
def test_forced_kernels_over_native_slabs(kernel: int, batch: int) -> None:
    """fk_w4a16_forward_kernel over native asymmetric slabs, both forced kernels."""
    from fast_kernels.ops import convert_arc_to_native_packets

    case = make_case(batch, 512, 32 * 128, 128, act="bf16", asymmetric=True, seed=77 + batch)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=128)
    slabs = convert_arc_to_native_packets(packets, n=512, k=4096, group_size=128,
                                          packet_format="native_asym")
    native = native_module()
    plan = arc_w4a16_plan(batch=batch, n=512, k=4096, group_size=128,
                          activation_dtype=torch.bfloat16, packet_format=2, kernel=kernel)
    ws = torch.zeros(max(1, plan["workspace_bytes"]) + 256, device=DEV, dtype=torch.uint8)
    y = torch.empty((batch, 512), device=DEV, dtype=torch.bfloat16)
    native.w4a16_forward_kernel(x.data_ptr(), slabs.data_ptr(), y.data_ptr(), ws.data_ptr(),
                                ws.numel(), batch, 512, 4096, 128, 2, 1, 0, kernel,
                                torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128, "bf16")
    _assert_gemv_close(_bits(y), ref, case, f"native kernel={kernel} M={batch}")


def test_forward_respects_current_stream() -> None:
    """Reference test_arc_kernel_respects_current_stream (:248-281)."""
    case = make_case(1, 128, 256, 128, seed=2112)
    x_expected, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=128)
    x = torch.zeros_like(x_expected)
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(50_000_000)
        x.copy_(x_expected)
        y = arc_w4a16_forward(x, packets, n=128, k=256, group_size=128)
    stream.synchronize()
    torch.cuda.synchronize()
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128)
    _assert_gemv_close(_bits(y), ref, case, "side stream")


def test_invalid_arguments_raise_value_error() -> None:
    case = make_case(1, 128, 256, 128)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=128)
    with pytest.raises(ValueError):
        arc_w4a16_forward(x, packets, n=128, k=256, group_size=96)
    with pytest.raises(ValueError):
        arc_w4a16_forward(x, packets[:1], n=128, k=256, group_size=128)
    with pytest.raises(ValueError):
        arc_w4a16_forward(x, packets, n=128, k=256, group_size=128, split_k_slices=0)


def test_reference_forward_on_two_streams_at_once() -> None:
    """The reference-signature arc_w4a16_forward (library-owned fix-up workspace) on two streams
    whose launches overlap: each stream has its own workspace, so both results match the oracle."""
    shapes = [(1, 4096, 14336, 128), (1, 1024, 16384, 128)]
    runs = []
    for batch, n, k, g in shapes:
        plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=g)
        assert plan["workspace_bytes"] > 0, plan
        case = make_case(batch, n, k, g, seed=n + k)
        x, q, a, b = _upload(case)
        runs.append((case, x, pack_arc_w4a16_packets(q, a, b, group_size=g)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    outs = []
    for _ in range(3):  # the first round allocates each stream's workspace
        outs = []
        for (case, x, packets), s in zip(runs, streams):
            y = torch.empty((1, case.n), device=DEV, dtype=torch.float16)
            with torch.cuda.stream(s):
                for _ in range(20):
                    native_module().arc_w4a16_forward(
                        x.data_ptr(), packets.data_ptr(), 0, y.data_ptr(), 1, case.n, case.k,
                        case.group_size, arc_packet_stride_bytes(case.group_size), s.cuda_stream)
            outs.append(y)
        torch.cuda.synchronize()
    for (case, _, _), y in zip(runs, outs):
        ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, case.group_size)
        _assert_gemv_close(_bits(y), ref, case, f"two streams {case.n}x{case.k}")
