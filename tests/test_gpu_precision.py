"""GPU precision tests whose bar scales with the activations.

The GEMV bar of the other parity tests, |err| <= 1e-2 |y| + 1e-2 sqrt(K) max|alpha|, has an
absolute term that does not shrink with x, so activations scaled far down (or wide-ranging ones)
would pass whatever the relative error. Here every output is held to

    |y - y_ref| <= ulp(y_ref) + 1e-3 * sum_k |W[n, k]| |x[m, k]|

with W = alpha * q + beta in float64 and y_ref the oracle's double-accumulated result rounded once
to the output dtype: one output ulp for the final rounding, plus 1e-3 of the magnitude of the terms
that were summed (fp32 accumulation of products of exact fp16 values stays near 1e-6 of it).
Activations are N(0, 1) scaled by powers of two from 2^-40 to 2^40 (within each dtype's range),
and "mixed": |x| = 2^u, u uniform over 30 binades, random signs, so that one group holds values
2^30 apart. Every packet format (reference packets, native symmetric and asymmetric slabs) and
both kernels (the dot2 loop at 1 and 4 rows, the matrix cores at 16) are run, and the stream
schedules of larger shapes (packet eighths, the matrix cores over packet quarters, K in parts).
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

from fast_kernels.benchmarking.inputs import bf16_bits_to_f32, f16_bits_to_f32, f32_to_bf16_bits, make_case  # noqa: E402
from fast_kernels.native import native_module  # noqa: E402
from fast_kernels.ops import (  # noqa: E402
    arc_w4a16_plan,
    convert_arc_to_native_packets,
    pack_arc_w4a16_packets,
)
from oracle import oracle  # noqa: E402
from test_gpu_w4a16_parity import _bits, _upload  # noqa: E402

DEV = "cuda"
N, K = 256, 1024

SCALES = {
    "f16": ["2^-12", "2^-20", "2^6", "mixed"],
    "bf16": ["2^-12", "2^-40", "2^8", "2^40", "mixed"],
}


def _scaled_x(case, scale: str) -> np.ndarray:
    rng = np.random.default_rng(case.seed + 17)
    shape = case.x.shape
    if scale == "mixed":
        lo, hi = (-20, 10) if case.act == "f16" else (-40, 30)
        mag = np.exp2(rng.uniform(lo, hi, size=shape))
        x = (mag * np.where(rng.random(shape) < 0.5, -1.0, 1.0)).astype(np.float32)
    else:
        e = int(scale.split("^")[1])
        x = (rng.standard_normal(shape) * 2.0**e).astype(np.float32)
    if case.act == "f16":
        return x.astype(np.float16).view(np.uint16)
    return f32_to_bf16_bits(x)


def _weights_f64(case) -> np.ndarray:
    lo = (case.q_u8 & 0xF).astype(np.float64)
    hi = (case.q_u8 >> 4).astype(np.float64)
    q = np.empty((case.n, case.k), dtype=np.float64)
    q[:, 0::2] = lo
    q[:, 1::2] = hi
    g = case.group_size
    a = np.repeat(f16_bits_to_f32(case.alpha).astype(np.float64), g, axis=1)
    b = np.repeat(f16_bits_to_f32(case.beta).astype(np.float64), g, axis=1)
    return a * q + b


def _ulp(ref: np.ndarray, act: str) -> np.ndarray:
    if act == "f16":
        return np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    mag = np.maximum(np.abs(ref), 2.0**-126)
    return np.exp2(np.floor(np.log2(mag)) - 7)


def _run(case, fmt: int, kernel: int) -> np.ndarray:
    x, q, a, b = _upload(case)
    g = case.group_size
    packets = pack_arc_w4a16_packets(q, a, b, group_size=g)
    if fmt != 0:
        packets = convert_arc_to_native_packets(
            packets, n=case.n, k=case.k, group_size=g,
            packet_format="native_sym" if fmt == 1 else "native_asym",
        )
    act = 0 if case.act == "f16" else 1
    plan = arc_w4a16_plan(batch=case.batch, n=case.n, k=case.k, group_size=g,
                          activation_dtype=x.dtype, packet_format=fmt, kernel=kernel)
    ws = torch.zeros(max(1, plan["workspace_bytes"]) + 256, device=DEV, dtype=torch.uint8)
    y = torch.empty((case.batch, case.n), device=DEV, dtype=x.dtype)
    native_module().w4a16_forward_kernel(
        x.data_ptr(), packets.data_ptr(), y.data_ptr(), ws.data_ptr(), ws.numel(), case.batch,
        case.n, case.k, g, fmt, act, 0, kernel, torch.cuda.current_stream().cuda_stream,
    )
    torch.cuda.synchronize()
    return _bits(y)


@pytest.mark.parametrize("kernel,batch", [(1, 1), (1, 4), (2, 16)])
@pytest.mark.parametrize("fmt", [0, 1, 2])
@pytest.mark.parametrize("group_size", [64, 128])
@pytest.mark.parametrize("act,scale", [(a, s) for a, ss in SCALES.items() for s in ss])
def test_error_relative_to_term_magnitudes(act, scale, group_size, fmt, kernel, batch) -> None:
    case = make_case(batch, N, K, group_size, act=act, asymmetric=(fmt != 1),
                     seed=1000 + 7 * group_size + fmt)
    case.x[:] = _scaled_x(case, scale)
    y_bits = _run(case, fmt, kernel)
    ref_bits, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size, act)
    to_f32 = f16_bits_to_f32 if act == "f16" else bf16_bits_to_f32
    y = to_f32(y_bits).astype(np.float64)
    ref = to_f32(ref_bits).astype(np.float64)
    mag = np.abs(case.x_f32().astype(np.float64)) @ np.abs(_weights_f64(case)).T
    assert np.all(np.isfinite(y))
    err = np.abs(y - ref)
    bound = _ulp(ref, act) + 1e-3 * mag
    rel = float(np.max(err / np.maximum(mag, 1e-300)))
    worst = np.unravel_index(int(np.argmax(err - bound)), err.shape)
    assert np.all(err <= bound), (
        f"{act} x~{scale} G={group_size} fmt={fmt} kernel={kernel} M={batch}: "
        f"err {err[worst]:.4g} > bound {bound[worst]:.4g} at {worst} (ref {ref[worst]:.4g}, "
        f"sum|Wx| {mag[worst]:.4g}); max err/sum|Wx| = {rel:.3g}"
    )


# The stream schedules added for the reference packets and for long K, under the same bar:
# (batch, n, k, group size, packet format, (m_tile, slice_cols, K parts) of the automatic plan).
STREAM_CASES = [
    (1, 4096, 4096, 128, 0, (1, 16, 1)),   # one row by 16-column packet eighths
    (8, 4096, 4096, 64, 0, (16, 32, 1)),   # matrix cores over packet quarters, whole rows staged
    (4, 2048, 16384, 64, 0, (16, 32, 4)),  # the same with K in four parts
    (4, 2048, 16384, 64, 2, (16, 32, 4)),  # K in parts over native asymmetric slabs
]


@pytest.mark.parametrize("batch,n,k,group_size,fmt,want", STREAM_CASES)
@pytest.mark.parametrize("act,scale", [("f16", "2^-20"), ("f16", "mixed"), ("bf16", "2^-40"),
                                       ("bf16", "2^40"), ("bf16", "mixed")])
def test_stream_schedules_error_relative_to_term_magnitudes(act, scale, batch, n, k, group_size,
                                                            fmt, want) -> None:
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the plans are chosen for 256 CUs")
    case = make_case(batch, n, k, group_size, act=act, asymmetric=(fmt != 1),
                     seed=2000 + 7 * group_size + fmt + batch)
    case.x[:] = _scaled_x(case, scale)
    plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=group_size,
                          activation_dtype=torch.float16 if act == "f16" else torch.bfloat16,
                          packet_format=fmt)
    assert plan["schedule"] == 2, plan
    assert (plan["m_tile"], plan["slice_cols"], plan["max_tile_contributors"]) == want, plan
    y_bits = _run(case, fmt, 0)
    ref_bits, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, group_size, act)
    to_f32 = f16_bits_to_f32 if act == "f16" else bf16_bits_to_f32
    y = to_f32(y_bits).astype(np.float64)
    ref = to_f32(ref_bits).astype(np.float64)
    mag = np.abs(case.x_f32().astype(np.float64)) @ np.abs(_weights_f64(case)).T
    assert np.all(np.isfinite(y))
    err = np.abs(y - ref)
    bound = _ulp(ref, act) + 1e-3 * mag
    worst = np.unravel_index(int(np.argmax(err - bound)), err.shape)
    assert np.all(err <= bound), (
        f"{act} x~{scale} {n}x{k} G={group_size} fmt={fmt} M={batch} plan={plan}: "
        f"err {err[worst]:.4g} > bound {bound[worst]:.4g} at {worst} (ref {ref[worst]:.4g})"
    )
