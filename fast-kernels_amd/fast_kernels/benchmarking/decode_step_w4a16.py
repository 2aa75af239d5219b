"""Runner of the decode_step_w4a16 suite family: a sustained decode-step stream.

A stack of ``metadata.layers`` Llama-style layers, each with the suite's projection shapes
(qkv, o, gate_up, down) and its own seeded int4 weights, is laid out in HBM as ARC packets. All
GEMVs of one decode step (layers x projections) are captured in one HIP graph and replayed; the
step's weights (3.6 GB for the 32-layer 8B stack) exceed every cache, so each replay streams them
from HBM. Reported per suite shape: device microseconds per GEMV (a graph of that projection
over all layers) and, as the extra shape "decode_step", microseconds per whole step and aggregate
effective HBM GB/s. When the suite lists the native-slab kernel id, the same stack is converted to
native symmetric slabs and timed the same way, and two more shapes time the layers as a Llama block
chains them (input RMSNorms and the SiLU-and-multiply included): "decode_step_layers_unfused"
(torch norm and activation kernels between the GEMVs) and "decode_step_layers_fused" (the norm and
the activation fused into the GEMV launches). The torch reference baseline (dequantize + matmul
per GEMV) is timed eagerly.

Correctness: after the timed replays, the outputs of the first and the last layer are compared
with the explicit fp32 formula (alpha*q + beta weights, fp32 matmul) within the suite tolerances.

Weights and activations are drawn on the GPU from a seeded torch generator (codes U{0..15},
alpha U[0.001, 0.02], zero point 8 so beta = -8 alpha exactly, x ~ N(0, 1)): the benchmark
configuration's recipe, generated where it is used instead of copied from the host.
"""

from __future__ import annotations

import math
from statistics import median
from typing import Any

from fast_kernels.benchmarking.decode_linear_w4a16 import (
    PEAK_HBM_GBS,
    _case,
    _check_close,
    _explicit_reference,
    _max_err,
    _p95,
)
from fast_kernels.benchmarking.inputs import algorithmic_bytes, seed_for_case
from fast_kernels.schemas import BenchmarkCase, BenchmarkSuite

GRAPH_REPLAYS = 20
DEVICE_TIMING_BLOCKS = 5
REFERENCE_SUBJECT = "torch/reference_w4a16_linear"
STEP_SHAPE = "decode_step"


def _all(suite: BenchmarkSuite, status: str, reason: str) -> list[BenchmarkCase]:
    cases = []
    for dtype in suite.dtypes:
        for layout in suite.layouts:
            names = [s.name for s in suite.shapes] + [STEP_SHAPE]
            for name in names:
                dims = next((s.dimensions() for s in suite.shapes if s.name == name), {"batch": 1})
                for kind, ids in (("kernel", suite.kernels.ids), ("baseline", suite.baselines.ids)):
                    cases += [_case(kind, sid, dtype, layout, name, dims, status, reason=reason)
                              for sid in ids]
    return cases


def run_decode_step_w4a16_suite(suite: BenchmarkSuite) -> tuple[list[BenchmarkCase], list[str]]:
    layers = int(suite.metadata.get("layers", 32))
    notes = [
        f"{layers} layers x {len(suite.shapes)} projections, distinct seeded weights per layer, "
        "one HIP graph per measured stream, replays timed with HIP events.",
    ]
    try:
        import torch
    except ImportError:
        return _all(suite, "skipped", "PyTorch is not installed."), notes
    from fast_kernels.ops import hip_decode_available

    if not hip_decode_available():
        return _all(suite, "skipped", "Native module is not built with HIP support."), notes
    if not torch.cuda.is_available():
        return _all(suite, "skipped", "torch.cuda.is_available() is false on this machine."), notes
    cases: list[BenchmarkCase] = []
    for dtype in suite.dtypes:
        for layout in suite.layouts:
            cases += _run_stack(torch, suite, dtype, layout, layers)
    return cases, notes


def layer_weights(torch: Any, device: Any, n: int, k: int, group_size: int, layer: int) -> tuple:
    """One projection's int4 weights in one layer of the stack: (q_u8 [n, k/2], alpha fp16
    [n, k/G], beta = -8 alpha fp16), drawn on the device from a generator seeded by the case seed
    and the layer index, so that every layer is distinct and any layer can be rebuilt alone."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed_for_case(1, n, k, group_size) * 131 + layer)
    q = torch.randint(0, 256, (n, k // 2), dtype=torch.uint8, device=device, generator=gen)
    alpha = torch.empty((n, k // group_size), device=device).uniform_(0.001, 0.02, generator=gen).half()
    beta = (alpha.float() * -8.0).half()
    return q, alpha, beta


def step_activations(torch: Any, device: Any, ks: list[int], act_dtype: Any) -> dict[int, Any]:
    """The step's activation rows, one per distinct K, x ~ N(0, 1) in the activation dtype."""
    gen = torch.Generator(device=device)
    gen.manual_seed(12345)
    return {k: torch.randn((1, k), device=device, generator=gen).to(act_dtype) for k in sorted(set(ks))}


LAYER_UNFUSED = "decode_step_layers_unfused"
LAYER_FUSED = "decode_step_layers_fused"


def _time_layer_chain(torch: Any, layers: int, dims: dict, slabs: dict, xs: dict, group_size: int,
                      act_dtype: Any, stream: Any, time_graph: Any) -> dict[str, tuple[float, float]]:
    """The layers' projections chained as a Llama block runs them (the attention itself and the
    residual adds aside), over native slabs, in two versions captured as one graph each:
    unfused (torch RMSNorm before qkv and gate_up, torch SiLU-and-multiply after gate_up) and
    fused (the RMSNorm prologue of qkv; gate_up with its norm and activation in one launch)."""
    from fast_kernels.ops import (
        arc_w4a16_forward_native,
        arc_w4a16_forward_rmsnorm,
        arc_w4a16_forward_silu_mul,
    )

    hidden = dims["qkv"][1]
    inter = dims["down"][1]
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(4242)
    x = torch.randn((1, hidden), device=dev, generator=gen).to(act_dtype)
    w_attn = (0.5 + torch.rand(hidden, device=dev, generator=gen)).to(act_dtype)
    w_ffn = (0.5 + torch.rand(hidden, device=dev, generator=gen)).to(act_dtype)
    qkv_out = torch.empty((1, dims["qkv"][0]), device=dev, dtype=act_dtype)
    o_out = torch.empty((1, dims["o"][0]), device=dev, dtype=act_dtype)
    gu_out = torch.empty((1, dims["gate_up"][0]), device=dev, dtype=act_dtype)
    act_out = torch.empty((1, inter), device=dev, dtype=act_dtype)
    down_out = torch.empty((1, dims["down"][0]), device=dev, dtype=act_dtype)
    o_in = xs[dims["o"][1]]

    def rmsnorm(v: Any, w: Any) -> Any:
        vf = v.float()
        h = (vf * torch.rsqrt(vf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(act_dtype)
        return (w.float() * h.float()).to(act_dtype)

    def proj(v: Any, layer: int, name: str, out: Any) -> None:
        n, k = dims[name]
        arc_w4a16_forward_native(v, slabs[(layer, name)], n=n, k=k, group_size=group_size,
                                 packet_format="native_sym", output=out)

    def unfused() -> None:
        for layer in range(layers):
            proj(rmsnorm(x, w_attn), layer, "qkv", qkv_out)
            proj(o_in, layer, "o", o_out)
            proj(rmsnorm(x, w_ffn), layer, "gate_up", gu_out)
            g, u = gu_out[:, :inter].float(), gu_out[:, inter:].float()
            act_out.copy_((torch.nn.functional.silu(g).to(act_dtype).float() * u).to(act_dtype))
            proj(act_out, layer, "down", down_out)

    def fused() -> None:
        for layer in range(layers):
            n, k = dims["qkv"]
            arc_w4a16_forward_rmsnorm(x, w_attn, slabs[(layer, "qkv")], n=n, k=k,
                                      group_size=group_size, eps=1e-5, output=qkv_out)
            proj(o_in, layer, "o", o_out)
            n, k = dims["gate_up"]
            arc_w4a16_forward_silu_mul(x, slabs[(layer, "gate_up")], n=n, k=k,
                                       group_size=group_size, output=act_out, norm_weight=w_ffn,
                                       eps=1e-5)
            proj(act_out, layer, "down", down_out)

    results = {}
    for name, fn in ((LAYER_UNFUSED, unfused), (LAYER_FUSED, fused)):
        with torch.cuda.stream(stream):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            fn()
        results[name] = time_graph(graph)
    return results


def _run_stack(torch: Any, suite: BenchmarkSuite, dtype: str, layout: str, layers: int) -> list[BenchmarkCase]:
    from fast_kernels.ops import (
        arc_packet_stride_bytes,
        arc_w4a16_forward,
        arc_w4a16_forward_native,
        convert_arc_to_native_packets,
        dequant_w4a16_to_fp16,
        group_size_for_layout,
        pack_arc_w4a16_packets,
        packet_stride_bytes,
    )
    from fast_kernels.registry import kernel_registry

    act_dtype = {"fp16": torch.float16, "bf16": torch.bfloat16}.get(dtype)
    if act_dtype is None:
        return [c for c in _all(suite, "skipped", f"dtype {dtype!r} is not supported")
                if c.dtype == dtype and c.layout == layout]
    device = torch.device("cuda")
    group_size = group_size_for_layout(layout)
    atol, rtol = suite.tolerances.atol, suite.tolerances.rtol
    shapes = [(s.name, s.require_dimension("n"), s.require_dimension("k"), s.dimensions())
              for s in suite.shapes]
    layer_results: dict[str, tuple[float, float]] = {}
    registry = kernel_registry()
    native_id = next((kid for kid in suite.kernels.ids if registry[kid].impl == "native"), None)
    slabs: dict[tuple[int, str], Any] = {}
    try:
        weights: dict[tuple[int, str], tuple[Any, Any, Any, Any]] = {}
        keep_raw = {0, layers - 1}
        # Each format's weights of the whole stack in one allocation, as a loader places a model
        # (one allocation per weight between the generator's temporaries ran the 70B bench step
        # 0.7 % slower).
        arc_stride = arc_packet_stride_bytes(group_size)
        nat_stride = packet_stride_bytes(group_size, "native_sym")
        arc_rows = {name: (n // 128) * (k // group_size) for name, n, k, _ in shapes}
        nat_rows = {name: (n // 32) * (k // group_size) for name, n, k, _ in shapes}
        arc_pool = torch.empty(layers * sum(arc_rows.values()) * arc_stride, dtype=torch.uint8,
                               device=device)
        nat_pool = (torch.empty(layers * sum(nat_rows.values()) * nat_stride, dtype=torch.uint8,
                                device=device) if native_id is not None else None)
        arc_off = nat_off = 0
        for layer in range(layers):
            for name, n, k, _ in shapes:
                q, alpha, beta = layer_weights(torch, device, n, k, group_size, layer)
                nbytes = arc_rows[name] * arc_stride
                packets = pack_arc_w4a16_packets(
                    q, alpha, beta, group_size=group_size,
                    packets=arc_pool[arc_off:arc_off + nbytes].view(arc_rows[name], arc_stride))
                arc_off += nbytes
                weights[(layer, name)] = (packets, q, alpha, beta) if layer in keep_raw else (packets, None, None, None)
                if nat_pool is not None:
                    nbytes = nat_rows[name] * nat_stride
                    slabs[(layer, name)] = convert_arc_to_native_packets(
                        packets, n=n, k=k, group_size=group_size, packet_format="native_sym",
                        packets=nat_pool[nat_off:nat_off + nbytes].view(nat_rows[name], nat_stride))
                    nat_off += nbytes
        del arc_pool, nat_pool
        xs = step_activations(torch, device, [k for _, _, k, _ in shapes], act_dtype)
        outs = {(layer, name): torch.empty((1, n), device=device, dtype=act_dtype)
                for layer in range(layers) for name, n, _, _ in shapes}
        stream = torch.cuda.Stream()

        def launch(selection: list[str], native: bool = False) -> None:
            for layer in range(layers):
                for name, n, k, _ in shapes:
                    if name not in selection:
                        continue
                    if native:
                        arc_w4a16_forward_native(xs[k], slabs[(layer, name)], n=n, k=k,
                                                 group_size=group_size, packet_format="native_sym",
                                                 output=outs[(layer, name)])
                    else:
                        arc_w4a16_forward(xs[k], weights[(layer, name)][0], n=n, k=k,
                                          group_size=group_size, output=outs[(layer, name)])

        def graph_for(selection: list[str], native: bool = False) -> Any:
            with torch.cuda.stream(stream):
                launch(selection, native)  # warm-up: plans and the workspace exist before capture
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                launch(selection, native)
            return graph

        def time_graph(graph: Any) -> tuple[float, float]:
            with torch.cuda.stream(stream):
                for _ in range(2):
                    graph.replay()
                torch.cuda.synchronize()
                samples = []
                for _ in range(DEVICE_TIMING_BLOCKS):
                    start = torch.cuda.Event(enable_timing=True)
                    end = torch.cuda.Event(enable_timing=True)
                    start.record(stream)
                    for _ in range(GRAPH_REPLAYS):
                        graph.replay()
                    end.record(stream)
                    end.synchronize()
                    samples.append(start.elapsed_time(end) * 1e3 / GRAPH_REPLAYS)
            return float(median(samples)), _p95(samples)

        step_graph = graph_for([name for name, _, _, _ in shapes])
        step_med, step_p95 = time_graph(step_graph)
        # Check a replayed step: every output of the first and the last layer.
        errors: dict[str, float] = {}
        for layer in sorted(keep_raw):
            for name, n, k, _ in shapes:
                _, q, alpha, beta = weights[(layer, name)]
                ref = _explicit_reference(torch, xs[k], q, alpha, beta, group_size)
                _check_close(outs[(layer, name)], ref, atol, rtol, f"layer {layer} {name}")
                errors[name] = max(errors.get(name, 0.0), _max_err(outs[(layer, name)], ref))
        per_shape = {}
        for name, _, _, _ in shapes:
            per_shape[name] = time_graph(graph_for([name]))
        native_results: dict[str, tuple[float, float]] = {}
        native_errors: dict[str, float] = {}
        if native_id is not None:
            all_names = [name for name, _, _, _ in shapes]
            native_results[STEP_SHAPE] = time_graph(graph_for(all_names, native=True))
            for layer in sorted(keep_raw):
                for name, n, k, _ in shapes:
                    _, q, alpha, beta = weights[(layer, name)]
                    ref = _explicit_reference(torch, xs[k], q, alpha, beta, group_size)
                    _check_close(outs[(layer, name)], ref, atol, rtol, f"native layer {layer} {name}")
                    native_errors[name] = max(native_errors.get(name, 0.0),
                                              _max_err(outs[(layer, name)], ref))
            for name in all_names:
                native_results[name] = time_graph(graph_for([name], native=True))
            dims = {name: (n, k) for name, n, k, _ in shapes}
            if {"qkv", "o", "gate_up", "down"} <= set(dims) and dims["down"][1] * 2 == dims["gate_up"][0]:
                layer_results = _time_layer_chain(torch, layers, dims, slabs, xs, group_size,
                                                  act_dtype, stream, time_graph)
    except Exception as exc:  # noqa: BLE001 - reported as failed cases
        return [c.model_copy(update={"status": "failed", "reason": str(exc)})
                for c in _all(suite, "failed", "") if c.dtype == dtype and c.layout == layout]

    cases: list[BenchmarkCase] = []
    step_bytes = sum(algorithmic_bytes(1, n, k, group_size) * layers for _, n, k, _ in shapes)

    def emit(kernel_id: str, results: dict[str, tuple[float, float]], errs: dict[str, float]) -> None:
        for name, n, k, dims in shapes:
            med, p95 = results[name]
            alg = algorithmic_bytes(1, n, k, group_size)
            us = med / layers
            cases.append(_case("kernel", kernel_id, dtype, layout, name, dims, "ok",
                               latency_us_median=us, latency_us_p95=p95 / layers,
                               device_latency_us_median=us, device_latency_us_p95=p95 / layers,
                               throughput=1e6 / us, decode_tokens_per_second=1e6 / us,
                               metrics={"hbm_gbs": alg / us / 1e3,
                                        "pct_hbm_peak": 100 * alg / us / 1e3 / PEAK_HBM_GBS,
                                        "algorithmic_bytes": float(alg), "layers": float(layers),
                                        "max_abs_err": errs.get(name, math.nan)}))
        s_med, s_p95 = results[STEP_SHAPE]
        cases.append(_case("kernel", kernel_id, dtype, layout, STEP_SHAPE,
                           {"batch": 1, "layers": layers, "gemvs": layers * len(shapes)}, "ok",
                           latency_us_median=s_med, latency_us_p95=s_p95,
                           device_latency_us_median=s_med, device_latency_us_p95=s_p95,
                           throughput=1e6 / s_med, decode_tokens_per_second=1e6 / s_med,
                           metrics={"hbm_gbs": step_bytes / s_med / 1e3,
                                    "pct_hbm_peak": 100 * step_bytes / s_med / 1e3 / PEAK_HBM_GBS,
                                    "algorithmic_bytes": float(step_bytes),
                                    "us_per_step": s_med}))

    arc_id = next((kid for kid in suite.kernels.ids if kid != native_id), None)
    if arc_id is not None:
        emit(arc_id, dict(per_shape, **{STEP_SHAPE: (step_med, step_p95)}), errors)
    if native_id is not None:
        emit(native_id, native_results, native_errors)
        for shape_name, (med, p95) in layer_results.items():
            cases.append(_case("kernel", native_id, dtype, layout, shape_name,
                               {"batch": 1, "layers": layers}, "ok",
                               latency_us_median=med, latency_us_p95=p95,
                               device_latency_us_median=med, device_latency_us_p95=p95,
                               throughput=1e6 / med, decode_tokens_per_second=1e6 / med,
                               metrics={"hbm_gbs": step_bytes / med / 1e3,
                                        "pct_hbm_peak": 100 * step_bytes / med / 1e3 / PEAK_HBM_GBS,
                                        "us_per_step": med}))
    timed_ids = {arc_id, native_id}
    for kid in suite.kernels.ids:
        if kid not in timed_ids:
            cases += [_case("kernel", kid, dtype, layout, name, dims, "not_implemented",
                            reason="the decode-step stream times the automatic dispatch and the "
                                   "native slabs only")
                      for name, _, _, dims in shapes]

    # torch reference: dequantize + matmul for every GEMV of one step, eager, a few steps.
    for baseline_id in suite.baselines.ids:
        if baseline_id != REFERENCE_SUBJECT:
            cases += [_case("baseline", baseline_id, dtype, layout, name, dims, "not_implemented",
                            reason=f"{baseline_id} has no decode-step runner")
                      for name, _, _, dims in shapes]
            continue
        wbuf = {name: torch.empty((n, k), device=device, dtype=torch.float16) for name, n, k, _ in shapes}

        def ref_step() -> None:
            # Layer 0's weights stand in for every layer: the traffic per GEMV is the same.
            for _layer in range(layers):
                for name, n, k, _ in shapes:
                    _, q, alpha, beta = weights[(0, name)]
                    dequant_w4a16_to_fp16(q, alpha, beta, group_size=group_size, output=wbuf[name])
                    torch.mm(xs[k].float(), wbuf[name].t().float())

        ref_step()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(3):
            ref_step()
        end.record()
        end.synchronize()
        ref_us = start.elapsed_time(end) * 1e3 / 3
        cases.append(_case("baseline", baseline_id, dtype, layout, STEP_SHAPE,
                           {"batch": 1, "layers": layers}, "ok",
                           latency_us_median=ref_us, device_latency_us_median=ref_us,
                           throughput=1e6 / ref_us, decode_tokens_per_second=1e6 / ref_us,
                           metrics={"hbm_gbs": step_bytes / ref_us / 1e3}))
        for c in cases:
            if c.subject_kind == "kernel" and c.shape_name == STEP_SHAPE and c.status == "ok":
                c.speedup_vs = {baseline_id: ref_us / c.device_latency_us_median}
    return cases
