"""fk_w4a16_forward_noalloc (the entry point that allocates nothing) through the C ABI, against
fk_arc_w4a16_forward_native with a caller workspace: the same plan and kernels, so the outputs
must be identical bit for bit. Two calls in a row, the second with a smaller input, both on
shapes whose plans split slices across workgroups (so the fixed scratch array carries the
fix-up counters and partials), and again in reverse size order."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import gpu_available

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="needs a GPU"),
]

torch = pytest.importorskip("torch")

from fast_kernels.benchmarking.inputs import make_case  # noqa: E402
from fast_kernels.native import native_module  # noqa: E402
from fast_kernels.ops import arc_w4a16_plan, convert_arc_to_native_packets, pack_arc_w4a16_packets  # noqa: E402
from test_gpu_w4a16_parity import _bits, _upload  # noqa: E402

DEV = "cuda"
FK_NOALLOC_SCRATCH_BYTES = 8388608 + 65536


def _lib() -> ctypes.CDLL:
    native_module()  # loads libfk_w4a16.so next to the binding; ctypes gets the same instance
    from fast_kernels.paths import package_root

    lib = ctypes.CDLL(str(package_root() / "libfk_w4a16.so"))
    P, I = ctypes.c_void_p, ctypes.c_int
    lib.fk_w4a16_forward_noalloc.argtypes = [P, P, P, I, I, I, I, I, I, P]
    lib.fk_arc_w4a16_forward_native.argtypes = [P, P, P, P, ctypes.c_size_t, I, I, I, I, I, I, I, P]
    lib.fk_last_error.restype = ctypes.c_char_p
    return lib


def _inputs(batch, n, k, g, act, fmt, seed):
    case = make_case(batch, n, k, g, act=act, asymmetric=(fmt == 2), seed=seed)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=g)
    if fmt:
        packets = convert_arc_to_native_packets(packets, n=n, k=k, group_size=g,
                                                packet_format="native_sym" if fmt == 1 else "native_asym")
    return x, packets


def _both(lib, shape):
    batch, n, k, g, act, fmt = shape
    x, packets = _inputs(batch, n, k, g, act, fmt, seed=n + k + batch)
    act_code = 0 if act == "f16" else 1
    plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=g, activation_dtype=x.dtype,
                          packet_format=fmt)
    assert 0 < plan["workspace_bytes"] <= FK_NOALLOC_SCRATCH_BYTES, plan
    stream = torch.cuda.current_stream().cuda_stream
    y_ref = torch.empty((batch, n), device=DEV, dtype=x.dtype)
    ws = torch.zeros(plan["workspace_bytes"] + 256, device=DEV, dtype=torch.uint8)
    rc = lib.fk_arc_w4a16_forward_native(x.data_ptr(), packets.data_ptr(), y_ref.data_ptr(),
                                         ws.data_ptr(), ws.numel(), batch, n, k, g, fmt, act_code,
                                         0, stream)
    assert rc == 0, lib.fk_last_error()
    y = torch.full((batch, n), float("nan"), device=DEV, dtype=x.dtype)
    rc = lib.fk_w4a16_forward_noalloc(x.data_ptr(), packets.data_ptr(), y.data_ptr(), batch, n, k,
                                      g, fmt, act_code, stream)
    assert rc == 0, lib.fk_last_error()
    torch.cuda.synchronize()
    return _bits(y), _bits(y_ref)


# (batch, n, k, G, activation, packet format) -- each plan splits slices (a fix-up workspace)
LARGE = (1, 4096, 14336, 64, "bf16", 1)    # 128 slices, two runs of 112 groups each
SMALL = (1, 1024, 8192, 64, "f16", 2)      # 32 slices, K split in four, asymmetric slabs
BATCHED = (8, 8192, 4096, 64, "f16", 0)    # matrix cores over reference packets, 4.5 MB scratch
TAIL = (1, 10240, 8192, 128, "bf16", 1)    # stream schedule: a quarter of a left-over slice per CU


@pytest.mark.parametrize("order", [(LARGE, SMALL), (BATCHED, LARGE), (SMALL, BATCHED), (TAIL, LARGE)])
def test_noalloc_matches_forward_native_two_calls(order) -> None:
    lib = _lib()
    for shape in order:
        y, y_ref = _both(lib, shape)
        np.testing.assert_array_equal(y, y_ref, err_msg=f"{shape}")


def test_noalloc_rejects_invalid_arguments_before_device_work() -> None:
    lib = _lib()
    rc = lib.fk_w4a16_forward_noalloc(None, None, None, 1, 128, 256, 96, 1, 0, None)
    assert rc == 1 and b"group_size" in lib.fk_last_error()
    rc = lib.fk_w4a16_forward_noalloc(None, None, None, 1, 128, 256, 128, 7, 0, None)
    assert rc == 1 and b"packet_format" in lib.fk_last_error()
