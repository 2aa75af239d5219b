"""GPU tests of the fused decode-step neighbours over native slabs.

Pins:
  * SiLU-and-multiply: against the unfused pipeline built from this library's own plain forward
    over the same slabs (run for run the same fp32 sums, so the gate and up halves match bit for
    bit) followed by torch's SiLU and product in the activation dtype: equal up to one ulp of the
    output dtype (the exponential of the two SiLUs may differ in its last fp32 bit); and, within
    the GEMV bar, against the oracle's gate and up GEMVs combined in float64.
  * RMSNorm prologue: against the unfused pipeline (torch RMSNorm with the Llama rounding, then
    the plain forward) and against the oracle GEMV of x normalised in float64 then rounded to the
    activation dtype, within the GEMV bar (rel 1e-2, abs 1e-2 * sqrt(K) * max|alpha|).
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

from fast_kernels.benchmarking.inputs import bf16_bits_to_f32, f16_bits_to_f32, make_case  # noqa: E402
from fast_kernels.ops import (  # noqa: E402
    arc_w4a16_forward_native,
    arc_w4a16_forward_rmsnorm,
    arc_w4a16_forward_silu_mul,
    arc_w4a16_plan,
    convert_arc_to_native_packets,
    pack_arc_w4a16_packets,
)
from oracle import oracle  # noqa: E402
from test_gpu_w4a16_parity import _assert_gemv_close, _bits, _upload  # noqa: E402

DEV = "cuda"


def _slabs(case, asym: bool):
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=case.group_size)
    fmt = "native_asym" if asym else "native_sym"
    slabs = convert_arc_to_native_packets(packets, n=case.n, k=case.k, group_size=case.group_size,
                                          packet_format=fmt)
    return x, slabs, fmt


def _to_f32(bits: np.ndarray, act: str) -> np.ndarray:
    return f16_bits_to_f32(bits) if act == "f16" else bf16_bits_to_f32(bits)


def _round_act(v: np.ndarray, act: str) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32))
    return t.to(torch.float16 if act == "f16" else torch.bfloat16).float().numpy()


@pytest.mark.parametrize("act", ["f16", "bf16"])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("group_size,asym", [(128, False), (64, True)])
def test_silu_mul_matches_unfused_pipeline(act, batch, group_size, asym) -> None:
    n, k = 1024, 16 * group_size  # gate 512 rows, up 512 rows
    case = make_case(batch, n, k, group_size, act=act, asymmetric=asym, seed=500 + batch)
    x, slabs, fmt = _slabs(case, asym)
    fused = arc_w4a16_forward_silu_mul(x, slabs, n=n, k=k, group_size=group_size,
                                       packet_format=fmt)
    y = arc_w4a16_forward_native(x, slabs, n=n, k=k, group_size=group_size, packet_format=fmt,
                                 split_k_slices=1)
    g, u = y[:, : n // 2].float(), y[:, n // 2 :].float()
    ref = (torch.nn.functional.silu(g).to(x.dtype).float() * u).to(x.dtype)
    torch.cuda.synchronize()
    got, want = fused.float(), ref.float()
    if batch < 8:  # from 8 rows the plain forward runs on the matrix cores, a different sum order
        ulp = 2.0 ** (-10 if act == "f16" else -7)
        bound = ulp * want.abs() + 1e-6
        assert bool(((got - want).abs() <= bound).all()), (
            f"max |fused - unfused| {float((got - want).abs().max()):.4g}"
        )
        assert float((got == want).float().mean()) > 0.99

    # the oracle's gate and up GEMVs, combined in float64
    ref_bits, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size, act)
    yo = _to_f32(ref_bits, act).astype(np.float64)
    go, uo = yo[:, : n // 2], yo[:, n // 2 :]
    so = _round_act(go / (1.0 + np.exp(-go)), act).astype(np.float64)
    want_o = so * uo
    max_alpha = float(f16_bits_to_f32(case.alpha).max())
    atol = 1e-2 * np.sqrt(k) * max_alpha * (np.abs(uo).max() + np.abs(so).max() + 1.0)
    err = np.abs(got.cpu().numpy().astype(np.float64) - want_o)
    assert np.all(err <= atol + 2e-2 * np.abs(want_o)), f"max err {err.max():.4g} atol {atol:.4g}"


@pytest.mark.parametrize("batch", [1, 3])
@pytest.mark.parametrize("with_norm", [False, True])
def test_silu_mul_over_several_staging_chunks(batch, with_norm) -> None:
    """K = 80 groups: more than one staging chunk, so the up half cannot reuse the activations
    the gate half staged and restages them; against the unfused pipeline within the GEMV bar."""
    n, k, g = 1024, 80 * 128, 128
    case = make_case(batch, n, k, g, act="bf16", seed=1700 + batch)
    x, slabs, fmt = _slabs(case, False)
    w = None
    xin = x
    if with_norm:
        gen = torch.Generator(device="cpu").manual_seed(11)
        w = (0.5 + torch.rand(k, generator=gen)).to(x.dtype).to(DEV)
        xin = _hf_rmsnorm(x, w, 1e-6)
    fused = arc_w4a16_forward_silu_mul(x, slabs, n=n, k=k, group_size=g, norm_weight=w, eps=1e-6)
    y = arc_w4a16_forward_native(xin, slabs, n=n, k=k, group_size=g, packet_format=fmt)
    gate, up = y[:, : n // 2].float(), y[:, n // 2 :].float()
    ref = (torch.nn.functional.silu(gate).to(x.dtype).float() * up).to(x.dtype)
    torch.cuda.synchronize()
    got = fused.float().cpu().numpy().astype(np.float64)
    want = ref.float().cpu().numpy().astype(np.float64)
    max_alpha = float(f16_bits_to_f32(case.alpha).max())
    atol = 1e-2 * np.sqrt(k) * max_alpha * (np.abs(want).max() + 1.0)
    err = np.abs(got - want)
    assert np.all(err <= atol + 2e-2 * np.abs(want)), f"max err {err.max():.4g}"


def _hf_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """Llama RMSNorm rounding: round(w * round(x * rsqrt(mean(x^2) + eps)))."""
    xf = x.float()
    h = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    return (w.float() * h.float()).to(x.dtype)


@pytest.mark.parametrize("act", ["f16", "bf16"])
@pytest.mark.parametrize("batch", [1, 2, 5, 8, 16])
@pytest.mark.parametrize("shape,asym", [((1024, 2048, 128), False), ((512, 4096, 64), True),
                                        ((4096, 14336, 128), False)])
def test_rmsnorm_matches_unfused_pipeline_and_oracle(act, batch, shape, asym) -> None:
    n, k, group_size = shape
    if k > 8192 and batch > 2:
        pytest.skip("large-K case runs at one and two rows")
    case = make_case(batch, n, k, group_size, act=act, asymmetric=asym, seed=900 + batch)
    x, slabs, fmt = _slabs(case, asym)
    gen = torch.Generator(device="cpu").manual_seed(7 + batch)
    w = (0.5 + torch.rand(k, generator=gen)).to(x.dtype).to(DEV)
    eps = 1e-5
    fused = arc_w4a16_forward_rmsnorm(x, w, slabs, n=n, k=k, group_size=group_size, eps=eps,
                                      packet_format=fmt)
    xn = _hf_rmsnorm(x, w, eps)
    unfused = arc_w4a16_forward_native(xn, slabs, n=n, k=k, group_size=group_size,
                                       packet_format=fmt)
    torch.cuda.synchronize()
    # the normalised activations agree with torch's up to the last bit of a few elements, so the
    # two results agree within the GEMV bar
    _assert_gemv_close(_bits(fused), _bits(unfused), case, f"fused vs unfused {shape} M={batch}")

    # oracle: x normalised in float64, rounded as above, then the oracle GEMV
    xf = _to_f32(case.x, act).astype(np.float64)
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + eps)
    h = _round_act(xf * inv, act).astype(np.float64)
    xn_np = _round_act(w.float().cpu().numpy().astype(np.float64) * h, act)
    xn_bits = torch.from_numpy(xn_np).to(x.dtype).view(torch.int16).numpy().view(np.uint16)
    ref_bits, _ = oracle.gemv(xn_bits, case.q_u8, case.alpha, case.beta, group_size, act)
    _assert_gemv_close(_bits(fused), ref_bits, case, f"fused vs oracle {shape} M={batch}")


def test_rmsnorm_plan_keeps_rows_on_dot2_kernel() -> None:
    from fast_kernels.native import native_module

    native = native_module()
    plan = native.w4a16_plan_rmsnorm(16, 4096, 4096, 128, 0, 0, 0, 1)
    assert plan["m_tile"] == 8 and plan["slice_cols"] == 32
    assert arc_w4a16_plan(batch=16, n=4096, k=4096, group_size=128, packet_format=1)["m_tile"] == 16


def test_fused_ops_reject_reference_packets_and_bad_shapes() -> None:
    case = make_case(1, 512, 1024, 128, seed=1)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=128)
    with pytest.raises(ValueError):
        arc_w4a16_forward_silu_mul(x, packets, n=512, k=1024, group_size=128, packet_format="arc")
    slabs = convert_arc_to_native_packets(packets, n=512, k=1024, group_size=128)
    with pytest.raises(ValueError):  # n must cover whole gate and up tiles
        arc_w4a16_forward_silu_mul(x, slabs, n=384, k=1024, group_size=128)
    w = torch.ones(1024, device=DEV, dtype=x.dtype)
    with pytest.raises(ValueError):
        arc_w4a16_forward_rmsnorm(x, w, slabs, n=512, k=1024, group_size=128, eps=-1.0)


@pytest.mark.parametrize("act", ["f16", "bf16"])
@pytest.mark.parametrize("batch", [1, 2, 4])
def test_rmsnorm_silu_mul_matches_unfused_pipeline(act, batch) -> None:
    """A Llama block's norm, gate_up and SiLU in one launch, against torch RMSNorm followed by the
    fused SiLU-and-multiply without the prologue, and against the oracle."""
    n, k, g = 2048, 4096, 128
    case = make_case(batch, n, k, g, act=act, seed=1300 + batch)
    x, slabs, fmt = _slabs(case, False)
    gen = torch.Generator(device="cpu").manual_seed(3)
    w = (0.5 + torch.rand(k, generator=gen)).to(x.dtype).to(DEV)
    fused = arc_w4a16_forward_silu_mul(x, slabs, n=n, k=k, group_size=g, norm_weight=w, eps=1e-6)
    xn = _hf_rmsnorm(x, w, 1e-6)
    unfused = arc_w4a16_forward_silu_mul(xn, slabs, n=n, k=k, group_size=g)
    torch.cuda.synchronize()
    got = fused.float().cpu().numpy().astype(np.float64)
    want = unfused.float().cpu().numpy().astype(np.float64)
    max_alpha = float(f16_bits_to_f32(case.alpha).max())
    atol = 1e-2 * np.sqrt(k) * max_alpha * (np.abs(want).max() + 1.0)
    err = np.abs(got - want)
    assert np.all(err <= atol + 2e-2 * np.abs(want)), f"max err {err.max():.4g}"
    assert np.mean(got == want) > 0.9  # the normalised activations rarely differ in a last bit


@pytest.mark.parametrize(
    "n,k,g,fuse",
    [
        (6144, 4096, 128, "rmsnorm"),         # Llama-8B qkv: 192 slices, one per workgroup
        (28672, 4096, 128, "rmsnorm_silu"),   # Llama-8B gate_up: 448 pairs, 2 per CU on 224 CUs
        (28672, 4096, 128, "silu"),
        (57344, 8192, 128, "silu"),           # Llama-70B gate_up: 896 pairs, 4 per CU on 224 CUs
        (16384, 4096, 64, "rmsnorm_silu"),    # G = 64: 256 pairs, one per CU
    ],
)
def test_stream_fused_one_row(n, k, g, fuse) -> None:
    """The fused neighbours on the stream kernel (one row, whole slices or gate/up slice pairs per
    workgroup): the RMSNorm prologue against torch's RMSNorm then the plain forward, and the SiLU
    epilogue against the plain forward then torch's SiLU and product (the same kernel's sums, so
    equal up to one ulp), and both against the oracle on a spread of columns."""
    from fast_kernels.native import native_module

    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    act = "bf16"
    case = make_case(1, n, k, g, act=act, seed=2100 + n // 1024 + k)
    x, slabs, fmt = _slabs(case, False)
    norm = fuse.startswith("rmsnorm")
    w = None
    xin = x
    eps = 1e-5
    if norm:
        gen = torch.Generator(device="cpu").manual_seed(5)
        w = (0.5 + torch.rand(k, generator=gen)).to(x.dtype).to(DEV)
        xin = _hf_rmsnorm(x, w, eps)
    native = native_module()
    if fuse == "rmsnorm":
        plan = native.w4a16_plan_rmsnorm(1, n, k, g, 1, 0, 0, 1)
        assert plan["schedule"] == 2, plan
        got = arc_w4a16_forward_rmsnorm(x, w, slabs, n=n, k=k, group_size=g, eps=eps,
                                        packet_format=fmt)
        want = arc_w4a16_forward_native(xin, slabs, n=n, k=k, group_size=g, packet_format=fmt)
        torch.cuda.synchronize()
        _assert_gemv_close(_bits(got), _bits(want), case, f"stream rmsnorm {n}x{k}")
        assert float((got == want).float().mean()) > 0.9
        xn_bits = xin.view(torch.int16).cpu().numpy().view(np.uint16)
        cols = np.unique(np.linspace(0, n - 1, 96).astype(int))
        ref, _ = oracle.gemv(xn_bits, np.ascontiguousarray(case.q_u8[cols]),
                             np.ascontiguousarray(case.alpha[cols]),
                             np.ascontiguousarray(case.beta[cols]), g, act)
        _assert_gemv_close(_bits(got)[:, cols], ref, case, f"stream rmsnorm vs oracle {n}x{k}")
        return
    got = arc_w4a16_forward_silu_mul(x, slabs, n=n, k=k, group_size=g, norm_weight=w, eps=eps)
    y = arc_w4a16_forward_native(xin, slabs, n=n, k=k, group_size=g, packet_format=fmt)
    gate, up = y[:, : n // 2].float(), y[:, n // 2 :].float()
    want = (torch.nn.functional.silu(gate).to(x.dtype).float() * up).to(x.dtype)
    torch.cuda.synchronize()
    gotf, wantf = got.float(), want.float()
    ulp = 2.0 ** -7
    if norm:
        # the row's 1 / rms may differ from torch's in a last bit: within the GEMV bar
        max_alpha = float(f16_bits_to_f32(case.alpha).max())
        atol = 1e-2 * np.sqrt(k) * max_alpha * (float(wantf.abs().max()) + 1.0)
        err = (gotf - wantf).abs()
        assert bool((err <= atol + 2e-2 * wantf.abs()).all()), f"max err {float(err.max()):.4g}"
        assert float((gotf == wantf).float().mean()) > 0.9
    else:
        assert bool(((gotf - wantf).abs() <= ulp * wantf.abs() + 1e-6).all())
        assert float((gotf == wantf).float().mean()) > 0.99
    # the oracle's gate and up GEMVs (a spread of output columns), combined in float64
    cols = np.unique(np.linspace(0, n // 2 - 1, 64).astype(int))
    both = np.concatenate([cols, cols + n // 2])
    xb = xin.view(torch.int16).cpu().numpy().view(np.uint16)
    ref_bits, _ = oracle.gemv(xb, np.ascontiguousarray(case.q_u8[both]),
                              np.ascontiguousarray(case.alpha[both]),
                              np.ascontiguousarray(case.beta[both]), g, act)
    yo = _to_f32(ref_bits, act).astype(np.float64)
    go, uo = yo[:, : cols.size], yo[:, cols.size :]
    so = _round_act(go / (1.0 + np.exp(-go)), act).astype(np.float64)
    want_o = so * uo
    max_alpha = float(f16_bits_to_f32(case.alpha).max())
    atol = 1e-2 * np.sqrt(k) * max_alpha * (np.abs(uo).max() + np.abs(so).max() + 1.0)
    err = np.abs(got[:, cols].float().cpu().numpy().astype(np.float64) - want_o)
    assert np.all(err <= atol + 2e-2 * np.abs(want_o)), f"max err {err.max():.4g}"
