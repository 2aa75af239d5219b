"""GPU parity at the benchmark configurations' exact shapes, against the CPU oracle.

  * configuration 1 (Llama-7B projections, M = 1, fp16): the four shapes over native symmetric
    slabs with the automatic plan, every row;
  * configuration 2 (Llama-70B layer, M = 1, bf16): the four projections over native symmetric
    slabs with the automatic plan, i.e. exactly the launches bench.py times (the stream schedule
    for o, gate_up and down, per-slice runs for qkv), and over the reference packets;
  * configuration 3 (N = 14336, K = 4096, G = 64, asymmetric, fp16, M = 2, 4, 8, 16): the
    automatic dispatch and both forced kernels (dot2 loop, matrix cores), over the reference
    packets and the native asymmetric slabs, every output against the oracle;
  * configuration 4 (the 32-layer Llama-8B decode step, bf16): the stack built as the
    decode-step runner builds it (distinct seeded weights per layer, native slabs), all 128
    GEMVs captured in one HIP graph and replayed twice, the outputs of layers 0, 15 and 31 of
    every projection against the oracle.

Like the reference's suite runner (decode_linear_w4a16.py:497-521), which gates every shape on
the explicit formula before timing it. Bar: the GEMV bar of the other parity tests
(rel 1e-2, abs 1e-2 * sqrt(K) * max|alpha|, test_gpu_w4a16_parity._assert_gemv_close).
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from conftest import gpu_available

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="needs a GPU"),
]

torch = pytest.importorskip("torch")

from fast_kernels.benchmarking.decode_step_w4a16 import layer_weights, step_activations  # noqa: E402
from fast_kernels.benchmarking.inputs import make_case  # noqa: E402
from fast_kernels.native import native_module  # noqa: E402
from fast_kernels.ops import (  # noqa: E402
    arc_w4a16_forward_native,
    arc_w4a16_plan,
    convert_arc_to_native_packets,
    pack_arc_w4a16_packets,
)
from oracle import oracle  # noqa: E402
from test_gpu_w4a16_parity import _assert_gemv_close, _bits, _upload  # noqa: E402

DEV = "cuda"

LLAMA70B = [("qkv", 10240, 8192), ("o", 8192, 8192), ("gate_up", 57344, 8192),
            ("down", 8192, 28672)]
LLAMA8B = [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096),
           ("down", 4096, 14336)]


def _rows(n: int) -> np.ndarray:
    """Every row up to 10240; for the larger shapes the first and last 1024 rows and 2048 spread
    between (each 32-column slice of a stream workgroup's range is covered at both ends)."""
    if n <= 10240:
        return np.arange(n)
    mid = np.linspace(1024, n - 1025, 2048).astype(int)
    return np.unique(np.concatenate([np.arange(1024), mid, np.arange(n - 1024, n)]))


def _oracle_rows(case, rows: np.ndarray, act: str) -> np.ndarray:
    ref, _ = oracle.gemv(case.x, np.ascontiguousarray(case.q_u8[rows]),
                         np.ascontiguousarray(case.alpha[rows]),
                         np.ascontiguousarray(case.beta[rows]), case.group_size, act)
    return ref


@pytest.mark.parametrize("packets", ["native_sym", "arc"])
@pytest.mark.parametrize("name,n,k", LLAMA70B)
def test_config2_llama70b_bf16_as_benchmarked(name: str, n: int, k: int, packets: str) -> None:
    case = make_case(1, n, k, 128, act="bf16")
    x, q, a, b = _upload(case)
    arc = pack_arc_w4a16_packets(q, a, b, group_size=128)
    code = 1 if packets == "native_sym" else 0
    slabs = arc if code == 0 else convert_arc_to_native_packets(arc, n=n, k=k, group_size=128)
    plan = arc_w4a16_plan(batch=1, n=n, k=k, group_size=128, activation_dtype=torch.bfloat16,
                          packet_format=code)
    if code == 1 and torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert plan["schedule"] == 2, plan  # qkv: 320 slices, one and a quarter per CU
    y = arc_w4a16_forward_native(x, slabs, n=n, k=k, group_size=128, packet_format=packets)
    torch.cuda.synchronize()
    rows = _rows(n)
    _assert_gemv_close(_bits(y)[:, rows], _oracle_rows(case, rows, "bf16"), case,
                       f"70B {name} {packets} plan={plan}")


LLAMA7B = [("qkv", 12288, 4096), ("o", 4096, 4096), ("gate_up", 22016, 4096),
           ("down", 4096, 11008)]


@pytest.mark.parametrize("name,n,k", LLAMA7B)
def test_config1_llama7b_fp16_as_suite_times(name: str, n: int, k: int) -> None:
    """Configuration 1 (Llama-7B projections, M = 1, G = 128, fp16) over native symmetric slabs
    with the automatic plan, the launches `fk bench` times for the 7B suite (half slices for o and
    down, per-slice runs or the stream schedule for qkv and gate_up): every output row against
    the oracle, and identical bits over three calls."""
    case = make_case(1, n, k, 128, act="f16")
    x, q, a, b = _upload(case)
    slabs = convert_arc_to_native_packets(pack_arc_w4a16_packets(q, a, b, group_size=128), n=n,
                                          k=k, group_size=128)
    plan = arc_w4a16_plan(batch=1, n=n, k=k, group_size=128, activation_dtype=torch.float16,
                          packet_format=1)
    outs = []
    for _ in range(3):
        y = arc_w4a16_forward_native(x, slabs, n=n, k=k, group_size=128, packet_format="native_sym")
        torch.cuda.synchronize()
        outs.append(_bits(y))
    ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 128, "f16")
    _assert_gemv_close(outs[0], ref, case, f"7B {name} native_sym plan={plan}")
    np.testing.assert_array_equal(outs[1], outs[0])
    np.testing.assert_array_equal(outs[2], outs[0])


_CONFIG3_REF: dict[int, tuple] = {}


def _config3_case(batch: int):
    if batch not in _CONFIG3_REF:
        case = make_case(batch, 14336, 4096, 64, act="f16", asymmetric=True)
        ref, _ = oracle.gemv(case.x, case.q_u8, case.alpha, case.beta, 64, "f16")
        _CONFIG3_REF.clear()
        _CONFIG3_REF[batch] = (case, ref)
    return _CONFIG3_REF[batch]


@pytest.mark.parametrize("batch", [2, 4, 8, 16])
@pytest.mark.parametrize("kernel", [0, 1, 2])  # automatic, dot2 loop, matrix cores
@pytest.mark.parametrize("packets", ["native_asym", "arc"])
def test_config3_small_batch_every_kernel(batch: int, kernel: int, packets: str) -> None:
    case, ref = _config3_case(batch)
    n, k, g = 14336, 4096, 64
    x, q, a, b = _upload(case)
    arc = pack_arc_w4a16_packets(q, a, b, group_size=g)
    code = 2 if packets == "native_asym" else 0
    slabs = arc if code == 0 else convert_arc_to_native_packets(arc, n=n, k=k, group_size=g,
                                                                packet_format="native_asym")
    plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=g, activation_dtype=torch.float16,
                          packet_format=code, kernel=kernel)
    ws = torch.zeros(max(1, plan["workspace_bytes"]) + 256, device=DEV, dtype=torch.uint8)
    y = torch.empty((batch, n), device=DEV, dtype=torch.float16)
    native_module().w4a16_forward_kernel(
        x.data_ptr(), slabs.data_ptr(), y.data_ptr(), ws.data_ptr(), ws.numel(), batch, n, k, g,
        code, 0, 0, kernel, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    _assert_gemv_close(_bits(y), ref, case, f"config 3 M={batch} kernel={kernel} {packets}")


def test_config4_llama8b_decode_step_graph() -> None:
    layers, g = 32, 128
    dev = torch.device(DEV)
    checked = (0, 15, 31)
    slabs, host = {}, {}
    for layer in range(layers):
        for name, n, k in LLAMA8B:
            q, alpha, beta = layer_weights(torch, dev, n, k, g, layer)
            arc = pack_arc_w4a16_packets(q, alpha, beta, group_size=g)
            slabs[(layer, name)] = convert_arc_to_native_packets(arc, n=n, k=k, group_size=g)
            if layer in checked:
                host[(layer, name)] = (q.cpu().numpy(), alpha.cpu().view(torch.int16).numpy().view(np.uint16),
                                       beta.cpu().view(torch.int16).numpy().view(np.uint16))
            del arc, q, alpha, beta
    xs = step_activations(torch, dev, [k for _, _, k in LLAMA8B], torch.bfloat16)
    outs = {(layer, name): torch.empty((1, n), device=dev, dtype=torch.bfloat16)
            for layer in range(layers) for name, n, _ in LLAMA8B}

    def step() -> None:
        for layer in range(layers):
            for name, n, k in LLAMA8B:
                arc_w4a16_forward_native(xs[k], slabs[(layer, name)], n=n, k=k, group_size=g,
                                         packet_format="native_sym", output=outs[(layer, name)])

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        step()  # eager warm-up: plans and workspaces exist before capture
    torch.cuda.synchronize()
    eager = {key: _bits(outs[key]) for key in host}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    for replay in range(2):
        for o in outs.values():
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for (layer, name), (q, alpha, beta) in host.items():
            n, k = next((n, k) for nm, n, k in LLAMA8B if nm == name)
            x_bits = _bits(xs[k])
            ref, _ = oracle.gemv(x_bits, q, alpha, beta, g, "bf16")
            c = SimpleNamespace(act="bf16", k=k, alpha=alpha)  # the fields the GEMV bar reads
            got = _bits(outs[(layer, name)])
            _assert_gemv_close(got, ref, c, f"8B step replay {replay} layer {layer} {name}")
            np.testing.assert_array_equal(got, eager[(layer, name)])


@pytest.mark.parametrize("packets", ["native_sym", "arc"])
def test_config2_layer_graph_replays_match_eager(packets: str) -> None:
    """The 70B layer captured in one HIP graph (native slabs: qkv takes pieces with a counter
    hand-off, the other three whole slices; reference packets: qkv pieces of packet quarters,
    gate_up whole tiles with pieces): four replays, with eager work and synchronisations between
    them, each bit-identical to the eager call (the counters the pieces leave behind are zero)."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the plans are chosen for 256 CUs")
    from fast_kernels.ops import arc_w4a16_forward

    dev = torch.device(DEV)
    weights, xs, outs = {}, {}, {}
    for name, n, k in LLAMA70B:
        q, alpha, beta = layer_weights(torch, dev, n, k, 128, 7)
        arc = pack_arc_w4a16_packets(q, alpha, beta, group_size=128)
        weights[name] = (arc if packets == "arc"
                         else convert_arc_to_native_packets(arc, n=n, k=k, group_size=128))
        del arc, q, alpha, beta
        xs[name] = torch.randn((1, k), device=dev).to(torch.bfloat16)
        outs[name] = torch.empty((1, n), device=dev, dtype=torch.bfloat16)
    for n in (10240, 57344):
        plan = arc_w4a16_plan(batch=1, n=n, k=8192, group_size=128,
                              activation_dtype=torch.bfloat16,
                              packet_format=0 if packets == "arc" else 1)
        assert plan["schedule"] == 2, plan
    plan = arc_w4a16_plan(batch=1, n=10240, k=8192, group_size=128,
                          activation_dtype=torch.bfloat16,
                          packet_format=0 if packets == "arc" else 1)
    assert plan["workspace_bytes"] > 0, plan

    def layer() -> None:
        for name, n, k in LLAMA70B:
            if packets == "arc":
                arc_w4a16_forward(xs[name], weights[name], n=n, k=k, group_size=128,
                                  output=outs[name])
            else:
                arc_w4a16_forward_native(xs[name], weights[name], n=n, k=k, group_size=128,
                                         packet_format="native_sym", output=outs[name])

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        layer()
    torch.cuda.synchronize()
    eager = {name: _bits(o) for name, o in outs.items()}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        layer()
    for replay in range(4):
        for o in outs.values():
            o.fill_(float("nan"))
        scratch = torch.randn(1 << 20, device=dev).sum()  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        del scratch
        for name, o in outs.items():
            np.testing.assert_array_equal(_bits(o), eager[name], err_msg=f"replay {replay} {name}")


@pytest.mark.parametrize(
    "n,k,g,act,asym,m",
    [
        (8192, 2048, 128, "f16", False, 1),  # 16 groups: one block of 8 waves x 2 slabs per slice
        (8192, 4096, 64, "f16", True, 1),      # G = 64: 4 slabs in flight per wave, two blocks
        (16384, 8192, 128, "bf16", True, 1),   # two whole slices per workgroup, asymmetric
        (8192, 32768, 128, "bf16", False, 1),  # the longest K the stream schedule stages
        (8192, 32768, 64, "f16", False, 1),    # 512 groups at G = 64
        # pieces of the slices left over past whole ones per CU, finished through the workspace
        (10240, 8192, 128, "bf16", False, 1),  # 1 slice + a quarter of one per CU
        (12288, 8192, 128, "f16", True, 1),    # 1 slice + a head and a tail piece (1.5 blocks)
        (12288, 4096, 64, "bf16", False, 1),   # G = 64: halves of 64 groups
        (10240, 16384, 64, "f16", True, 1),    # G = 64: quarters of 256 groups
        (22016, 8192, 128, "f16", True, 1),    # ranges of 1 or 2 blocks over 176 slices
        # half slices (G = 128, at most half as many slices as CUs)
        (4096, 4096, 128, "bf16", False, 1),   # 8B o
        (4096, 14336, 128, "f16", True, 1),    # 8B down, asymmetric
        (1024, 2048, 128, "bf16", True, 1),    # 64 workgroups
        (12288, 4096, 128, "bf16", True, 1),   # 768 half-slices, 3 per CU (7B qkv)
        (16384, 4096, 128, "f16", False, 1),   # 1024 half-slices, 4 per CU
        (6144, 4096, 128, "f16", False, 1),  # one slice per workgroup, 192 workgroups
        # half slices whose last block is partial (K/G not a multiple of 16)
        (4096, 11008, 128, "f16", False, 1),   # 7B down: 86 groups
        (8192, 28800, 128, "bf16", True, 1),   # 225 groups, two half slices per CU
        # more slices than CUs, a divisor of them over at least 7/8 of the CUs: whole slices only
        (28672, 8192, 128, "bf16", False, 1),  # 896 slices: 4 per workgroup on 224 CUs
        (28672, 4096, 128, "bf16", True, 1),   # 8B gate_up, asymmetric
    ],
)
def test_stream_schedule_variants(n: int, k: int, g: int, act: str, asym: bool, m: int) -> None:
    """The stream schedule (whole slices per CU, pieces of the slices left over, half slices, one
    slice per workgroup) at both group sizes, both activation dtypes, both native formats and the
    staging slot counts; plus determinism."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    case = make_case(m, n, k, g, act=act, asymmetric=asym, seed=n + k + g + m)
    x, q, a, b = _upload(case)
    fmt = "native_asym" if asym else "native_sym"
    slabs = convert_arc_to_native_packets(pack_arc_w4a16_packets(q, a, b, group_size=g), n=n, k=k,
                                          group_size=g, packet_format=fmt)
    plan = arc_w4a16_plan(batch=m, n=n, k=k, group_size=g,
                          activation_dtype=x.dtype, packet_format=2 if asym else 1)
    assert plan["schedule"] == 2, plan
    # three calls: the pieces' hand-off leaves its counters at zero, and adds the parts in a fixed
    # order, so every call gives the same bits
    ys = [_bits(arc_w4a16_forward_native(x, slabs, n=n, k=k, group_size=g, packet_format=fmt))
          for _ in range(3)]
    np.testing.assert_array_equal(ys[0], ys[1])
    np.testing.assert_array_equal(ys[0], ys[2])
    rows = _rows(n)
    _assert_gemv_close(ys[0][:, rows], _oracle_rows(case, rows, act), case, f"stream {plan}")


@pytest.mark.parametrize(
    "m,n,k,g,act,asym",
    [
        (3, 12288, 4096, 128, "bf16", False),  # 1 slice + pieces, four-row staging
        (4, 14336, 4096, 64, "f16", True),     # configuration 3, four rows
        (8, 8192, 4096, 128, "bf16", True),    # whole slices, eight rows
        (7, 6144, 4096, 128, "f16", False),    # 192 slices: one per workgroup, an odd batch
        (5, 8192, 4096, 128, "bf16", False),   # eight-row staging, G = 128
        (8, 14336, 4096, 64, "bf16", True),    # configuration 3's shape in bf16, eight rows
        # 448 slices: two per workgroup on 224 of the CUs, no pieces, 2 to 16 rows
        (2, 14336, 4096, 64, "f16", True),     # configuration 3, two rows
        (16, 14336, 4096, 64, "f16", True),    # configuration 3, sixteen rows
        (13, 14336, 4096, 128, "bf16", False),  # sixteen-row staging at G = 128, an odd batch
    ],
)
def test_mfma_stream_variants(m: int, n: int, k: int, g: int, act: str, asym: bool) -> None:
    """The matrix-core kernel on the stream schedule (rows staged whole in LDS, pieces handed off
    by the control wave): both group sizes, dtypes and formats, odd batches; every row against the
    oracle on a spread of columns, and identical bits over three calls."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    case = make_case(m, n, k, g, act=act, asymmetric=asym, seed=3 * n + k + g + m)
    x, q, a, b = _upload(case)
    fmt = "native_asym" if asym else "native_sym"
    slabs = convert_arc_to_native_packets(pack_arc_w4a16_packets(q, a, b, group_size=g), n=n, k=k,
                                          group_size=g, packet_format=fmt)
    plan = arc_w4a16_plan(batch=m, n=n, k=k, group_size=g,
                          activation_dtype=x.dtype, packet_format=2 if asym else 1)
    assert plan["schedule"] == 2 and plan["m_tile"] == 16, plan
    ys = [_bits(arc_w4a16_forward_native(x, slabs, n=n, k=k, group_size=g, packet_format=fmt))
          for _ in range(3)]
    np.testing.assert_array_equal(ys[0], ys[1])
    np.testing.assert_array_equal(ys[0], ys[2])
    rows = _rows(n)
    _assert_gemv_close(ys[0][:, rows], _oracle_rows(case, rows, act), case, f"mfma stream {plan}")


@pytest.mark.parametrize(
    "m,n,k,g,act,want",
    [
        # m, n, k, G, activation, (workgroups, whole slices each) on 256 CUs
        (2, 14336, 4096, 64, "f16", (224, 2)),    # configuration 3: 448 quarters on 224 CUs
        (5, 14336, 4096, 64, "bf16", (224, 2)),   # eight-row staging, bf16
        (16, 14336, 4096, 64, "f16", (224, 2)),   # sixteen rows
        (3, 4096, 4096, 128, "bf16", (128, 1)),   # G = 128: fewer quarters than CUs, one each
        (13, 8192, 4096, 128, "f16", (256, 1)),   # G = 128, sixteen-row staging, an odd batch
        (8, 16384, 4096, 64, "bf16", (256, 2)),   # two quarters per CU on every CU
    ],
)
def test_reference_packets_mfma_stream(m: int, n: int, k: int, g: int, act: str, want) -> None:
    """The reference signature (arc_w4a16_forward, arc_w4a16.cu:687-707) at 2-16 rows over the
    reference packets on the matrix-core stream kernel (w4a16_gemm_mfma_stream.hip, packet
    quarters as slices, any fp16 beta): both group sizes and dtypes; sampled rows of every output
    row against the oracle, and identical bits over three calls."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    from fast_kernels.ops import arc_w4a16_forward

    case = make_case(m, n, k, g, act=act, asymmetric=True, seed=5 * n + k + g + m)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=g)
    plan = arc_w4a16_plan(batch=m, n=n, k=k, group_size=g, activation_dtype=x.dtype,
                          packet_format=0)
    assert (plan["schedule"], plan["m_tile"], plan["slice_cols"]) == (2, 16, 32), plan
    assert (plan["workgroups"], plan["groups_per_workgroup"] // (k // g)) == want, plan
    outs = []
    for _ in range(3):
        y = arc_w4a16_forward(x, packets, n=n, k=k, group_size=g)
        torch.cuda.synchronize()
        outs.append(_bits(y))
    rows = _rows(n)
    _assert_gemv_close(outs[0][:, rows], _oracle_rows(case, rows, act), case,
                       f"reference packets, matrix-core stream, M={m} {n}x{k} G{g} {act} "
                       f"plan={plan}")
    np.testing.assert_array_equal(outs[1], outs[0])
    np.testing.assert_array_equal(outs[2], outs[0])


@pytest.mark.parametrize(
    "m,n,k,g,act,packets,parts",
    [
        (3, 4096, 14336, 64, "f16", "arc", 7),            # the MLP down shape: 7 parts of 32 groups
        (4, 4096, 14336, 64, "bf16", "native_asym", 7),
        (16, 4096, 14336, 64, "f16", "arc", 7),
        (5, 10240, 8192, 128, "f16", "arc", 4),           # 70B qkv: 4 parts of 16 groups, 5 slices
        (3, 8192, 8192, 128, "bf16", "arc", 2),           # 70B o: 2 parts, two slices per workgroup
        (8, 8192, 28672, 128, "bf16", "native_sym", 7),   # 70B down, 8 rows
    ],
)
def test_mfma_stream_k_parts(m: int, n: int, k: int, g: int, act: str, packets: str,
                             parts: int) -> None:
    """The matrix-core stream kernel with K in parts (rows too long to stage whole): each
    workgroup stages one part of K and streams whole slices over it, the parts' fp32 sums added in
    part order by a second launch. Both formats and dtypes, 2-16 rows; sampled rows against the
    oracle and identical bits over three calls."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    from fast_kernels.ops import arc_w4a16_forward

    asym = packets != "native_sym"
    case = make_case(m, n, k, g, act=act, asymmetric=asym, seed=7 * n + k + g + m)
    x, q, a, b = _upload(case)
    arc = pack_arc_w4a16_packets(q, a, b, group_size=g)
    code = {"arc": 0, "native_sym": 1, "native_asym": 2}[packets]
    weights = arc if code == 0 else convert_arc_to_native_packets(arc, n=n, k=k, group_size=g,
                                                                  packet_format=packets)
    plan = arc_w4a16_plan(batch=m, n=n, k=k, group_size=g, activation_dtype=x.dtype,
                          packet_format=code)
    assert (plan["schedule"], plan["m_tile"], plan["max_tile_contributors"]) == (2, 16, parts), plan

    def run():
        if code == 0:
            y = arc_w4a16_forward(x, weights, n=n, k=k, group_size=g)
        else:
            y = arc_w4a16_forward_native(x, weights, n=n, k=k, group_size=g, packet_format=packets)
        torch.cuda.synchronize()
        return _bits(y)

    outs = [run() for _ in range(3)]
    rows = _rows(n)
    _assert_gemv_close(outs[0][:, rows], _oracle_rows(case, rows, act), case,
                       f"matrix-core stream, {parts} K parts, M={m} {n}x{k} G{g} {act} {packets} "
                       f"plan={plan}")
    np.testing.assert_array_equal(outs[1], outs[0])
    np.testing.assert_array_equal(outs[2], outs[0])


def test_small_batch_stream_schedules_graph_replays_match_eager() -> None:
    """The 2-16-row matrix-core stream launches over the reference packets (whole rows staged,
    and K in parts: a GEMV launch and the parts' addition) captured in one HIP graph, replayed
    four times with eager work in between: every replay bit-identical to the eager run."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    from fast_kernels.ops import arc_w4a16_forward

    dev = torch.device(DEV)
    shapes = [(4, 14336, 4096, 64), (8, 4096, 14336, 64), (3, 8192, 28672, 128)]
    weights, xs, outs = {}, {}, {}
    for i, (m, n, k, g) in enumerate(shapes):
        case = make_case(m, n, k, g, act="f16", asymmetric=True, seed=300 + i)
        x, q, a, b = _upload(case)
        weights[i] = pack_arc_w4a16_packets(q, a, b, group_size=g)
        xs[i] = x
        outs[i] = torch.empty((m, n), device=dev, dtype=torch.float16)
        plan = arc_w4a16_plan(batch=m, n=n, k=k, group_size=g, activation_dtype=x.dtype,
                              packet_format=0)
        assert (plan["schedule"], plan["m_tile"]) == (2, 16), plan
        assert (plan["max_tile_contributors"] > 1) == (i > 0), plan

    def run() -> None:
        for i, (m, n, k, g) in enumerate(shapes):
            arc_w4a16_forward(xs[i], weights[i], n=n, k=k, group_size=g, output=outs[i])

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        run()  # the workspace exists before the capture
    torch.cuda.synchronize()
    eager = {i: _bits(o) for i, o in outs.items()}
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        run()
    for replay in range(4):
        for o in outs.values():
            o.fill_(float("nan"))
        scratch = torch.randn(1 << 20, device=dev).sum()  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        del scratch
        for i, o in outs.items():
            np.testing.assert_array_equal(_bits(o), eager[i], err_msg=f"replay {replay} {shapes[i]}")


@pytest.mark.parametrize(
    "n,k,g,act",
    [
        (32768, 4096, 128, "f16"),   # 256 tiles: one whole tile per CU, no pieces
        (65536, 8192, 128, "bf16"),  # two whole tiles per CU
        (57344, 8192, 128, "bf16"),  # 70B gate_up: two whole tiles per workgroup on 224 CUs
        (49152, 8192, 128, "f16"),   # 384 tiles: a whole tile and a piece of one per CU
        (40960, 2048, 64, "bf16"),   # G = 64 (blocks of 8 groups), pieces of a quarter tile
        (36864, 16384, 64, "f16"),   # G = 64, longer K (more staging passes), pieces
    ],
)
def test_reference_packets_stream_schedule(n: int, k: int, g: int, act: str) -> None:
    """The reference signature (arc_w4a16_forward, arc_w4a16.cu:687-707) over the reference
    packets on the stream schedule (w4a16_gemv_arc_stream.hip: whole 128-column tiles per
    workgroup, over a divisor grid or over every CU plus pieces): sampled rows against the oracle,
    and identical bits over three calls."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    from fast_kernels.ops import arc_w4a16_forward

    case = make_case(1, n, k, g, act=act, asymmetric=True, seed=n + k + g)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=g)
    plan = arc_w4a16_plan(batch=1, n=n, k=k, group_size=g, activation_dtype=x.dtype,
                          packet_format=0)
    assert plan["schedule"] == 2 and plan["slice_cols"] == 128, plan
    outs = []
    for _ in range(3):
        y = arc_w4a16_forward(x, packets, n=n, k=k, group_size=g)
        torch.cuda.synchronize()
        outs.append(_bits(y))
    rows = _rows(n)
    _assert_gemv_close(outs[0][:, rows], _oracle_rows(case, rows, act), case,
                       f"reference packets, stream schedule, {n}x{k} G{g} {act} plan={plan}")
    np.testing.assert_array_equal(outs[1], outs[0])
    np.testing.assert_array_equal(outs[2], outs[0])


@pytest.mark.parametrize(
    "n,k,g,act,want",
    [
        # n, k, G, activation, (unit columns, workgroups, groups per workgroup, fix-up
        # workspace) on 256 CUs
        (8192, 8192, 128, "bf16", (32, 256, 64, False)),    # 70B o: one 32-column slice per CU
        (10240, 8192, 128, "bf16", (32, 256, 80, True)),    # 70B qkv: a slice and a piece per CU
        (8192, 28672, 128, "bf16", (32, 256, 224, False)),  # 70B down: seven staging passes
        (14336, 4096, 128, "f16", (32, 224, 64, False)),    # divisor grid: 448 slices on 224 CUs
        (16384, 4096, 64, "f16", (32, 256, 128, False)),    # G = 64: blocks of 32 groups
        (10240, 8192, 64, "bf16", (32, 256, 160, True)),    # G = 64 with pieces
        # 16-column eighths of the packets (G = 128)
        (4096, 4096, 128, "f16", (16, 256, 32, False)),     # 7B o: one eighth per CU
        (2048, 4096, 128, "bf16", (16, 128, 32, False)),    # 128 eighths, one each
        (4096, 4096, 128, "bf16", (16, 256, 32, False)),    # 8B o
    ],
)
def test_reference_packets_quarter_schedule(n: int, k: int, g: int, act: str, want) -> None:
    """The reference signature (arc_w4a16_forward, arc_w4a16.cu:687-707) over the reference
    packets by 32-column quarters or 16-column eighths of the packets (w4a16_gemv_arc_quarter.hip),
    asymmetric packets (any fp16 beta): sampled rows against the oracle (every row for 7B o),
    identical bits over three calls."""
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("the shapes are chosen for 256 CUs")
    from fast_kernels.ops import arc_w4a16_forward

    case = make_case(1, n, k, g, act=act, asymmetric=True, seed=3 * n + k + g)
    x, q, a, b = _upload(case)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=g)
    plan = arc_w4a16_plan(batch=1, n=n, k=k, group_size=g, activation_dtype=x.dtype,
                          packet_format=0)
    assert plan["schedule"] == 2, plan
    got = (plan["slice_cols"], plan["workgroups"], plan["groups_per_workgroup"],
           plan["workspace_bytes"] > 0)
    assert got == want, plan
    outs = []
    for _ in range(3):
        y = arc_w4a16_forward(x, packets, n=n, k=k, group_size=g)
        torch.cuda.synchronize()
        outs.append(_bits(y))
    rows = np.arange(n) if n * k <= 4096 * 4096 else _rows(n)
    _assert_gemv_close(outs[0][:, rows], _oracle_rows(case, rows, act), case,
                       f"reference packets, quarter schedule, {n}x{k} G{g} {act} plan={plan}")
    np.testing.assert_array_equal(outs[1], outs[0])
    np.testing.assert_array_equal(outs[2], outs[0])
