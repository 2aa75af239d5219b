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
BATCHED = (8, 8192, 8192, 64, "f16", 0)    # matrix-core tiles over reference packets, 4.6 MB scratch
TAIL = (1, 10240, 8192, 128, "bf16", 1)    # stream schedule: a quarter of a left-over slice per CU
ARC_TAIL = (1, 10240, 8192, 128, "bf16", 0)  # reference packets by 32-column quarters, pieces


@pytest.mark.parametrize("order", [(LARGE, SMALL), (BATCHED, LARGE), (SMALL, BATCHED), (TAIL, LARGE),
                                   (ARC_TAIL, SMALL)])
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


def _noalloc(lib, x, packets, y, shape, stream):
    batch, n, k, g, act, fmt = shape
    return lib.fk_w4a16_forward_noalloc(x.data_ptr(), packets.data_ptr(), y.data_ptr(), batch, n,
                                        k, g, fmt, 0 if act == "f16" else 1, stream)


def test_noalloc_graph_capture_replays_match_eager() -> None:
    """A noalloc call captured in a HIP graph (torch.cuda.CUDAGraph), replayed three times with
    eager work in between: every replay equals forward_native bit for bit."""
    lib = _lib()
    y_eager, y_ref = _both(lib, TAIL)  # eager noalloc against forward_native, same inputs below
    np.testing.assert_array_equal(y_eager, y_ref)
    batch, n, k, g, act, fmt = TAIL
    x, packets = _inputs(batch, n, k, g, act, fmt, seed=n + k + batch)
    y = torch.full((batch, n), float("nan"), device=DEV, dtype=x.dtype)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=side):
            rc = _noalloc(lib, x, packets, y, TAIL, side.cuda_stream)
            assert rc == 0, lib.fk_last_error()
    torch.cuda.synchronize()
    for rep in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(y), y_ref, err_msg=f"replay {rep}")
        # eager work on the same scratch between replays
        y2 = torch.empty_like(y)
        assert _noalloc(lib, x, packets, y2, TAIL, torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        np.testing.assert_array_equal(_bits(y2), y_ref)


def test_noalloc_refuses_a_second_stream_while_the_first_is_busy() -> None:
    lib = _lib()
    batch, n, k, g, act, fmt = TAIL
    x, packets = _inputs(batch, n, k, g, act, fmt, seed=7)
    y = torch.empty((batch, n), device=DEV, dtype=x.dtype)
    a, b = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    assert _noalloc(lib, x, packets, y, TAIL, a.cuda_stream) == 0, lib.fk_last_error()
    with torch.cuda.stream(a):
        torch.cuda._sleep(200_000_000)  # a bounded spin: stream a has work queued for a while
    rc = _noalloc(lib, x, packets, y, TAIL, b.cuda_stream)
    busy = a.query() is False
    torch.cuda.synchronize()
    if busy:  # the spin was still running when b called (it takes tens of milliseconds)
        assert rc == 2 and b"still has work queued" in lib.fk_last_error(), rc
    # once stream a is idle, stream b takes the scratch over, and the results are unchanged
    y_b = torch.full_like(y, float("nan"))
    assert _noalloc(lib, x, packets, y_b, TAIL, b.cuda_stream) == 0, lib.fk_last_error()
    torch.cuda.synchronize()
    y_a = torch.full_like(y, float("nan"))
    assert _noalloc(lib, x, packets, y_a, TAIL, a.cuda_stream) == 0, lib.fk_last_error()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(y_a), _bits(y_b))


_FIRST_CALL_UNDER_CAPTURE = r"""
import sys
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import numpy as np
import torch
import test_zz_no_alloc as t

lib = t._lib()
batch, n, k, g, act, fmt = t.TAIL
x, packets = t._inputs(batch, n, k, g, act, fmt, seed=11)
torch.cuda.synchronize()
y = torch.full((batch, n), float("nan"), device="cuda", dtype=x.dtype)
side = torch.cuda.Stream()
with torch.cuda.stream(side):
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        rc = t._noalloc(lib, x, packets, y, t.TAIL, side.cuda_stream)  # the process's first call
assert rc == 0, lib.fk_last_error()
torch.cuda.synchronize()
outs = []
for _ in range(2):
    y.fill_(float("nan"))
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    outs.append(t._bits(y).copy())
plan = t.arc_w4a16_plan(batch=batch, n=n, k=k, group_size=g, activation_dtype=x.dtype,
                        packet_format=fmt)
ws = torch.zeros(plan["workspace_bytes"] + 256, device="cuda", dtype=torch.uint8)
y_ref = torch.empty_like(y)
rc = lib.fk_arc_w4a16_forward_native(x.data_ptr(), packets.data_ptr(), y_ref.data_ptr(),
                                     ws.data_ptr(), ws.numel(), batch, n, k, g, fmt,
                                     0 if act == "f16" else 1, 0,
                                     torch.cuda.current_stream().cuda_stream)
assert rc == 0, lib.fk_last_error()
torch.cuda.synchronize()
for o in outs:
    np.testing.assert_array_equal(o, t._bits(y_ref))
print("ok")
"""


def test_noalloc_first_call_of_the_process_under_graph_capture() -> None:
    """The device set-up (address lookup, clearing kernel) happening inside a capture: a fresh
    process whose first noalloc call is captured, replayed twice, equal to forward_native."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    tests_dir = Path(__file__).resolve().parent
    pkg = tests_dir.parent / "fast-kernels_amd"
    proc = subprocess.run(
        [sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, str(tests_dir), str(pkg)],
        capture_output=True, text=True, timeout=110, env=dict(os.environ),
        cwd=str(tests_dir.parent),
    )
    assert proc.returncode == 0 and "ok" in proc.stdout, proc.stdout[-2000:] + proc.stderr[-2000:]
