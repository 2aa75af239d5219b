"""Runner of the decode_linear_w4a16 suite family (``fk bench benchmarks/suites/decode_linear_*.toml``).

Same case matrix, case ids, statuses and gates as the reference runner
(src/fast_kernels/benchmarking/decode_linear_w4a16.py:292-684): every (dtype, layout, shape)
is first checked (reference baseline against the explicit fp32 formula, vendor baseline and every
kernel against the reference baseline, suite tolerances), then timed. Differences, all additive:

* dtypes "fp16" and "bf16" (bf16 activations and outputs; the vendor and tc paths are fp16-only
  and are skipped for bf16 with a reason);
* device time from HIP events around a HIP graph of back-to-back launches whose weights rotate
  through copies totalling >= 2 x 256 MiB, so every launch reads HBM rather than the 256 MB
  Infinity Cache and host launch overhead is excluded (``device_latency_us_*``); the
  reference's wall-clock-with-sync timing is kept as ``wall_latency_us_*``;
* metrics: effective HBM GB/s and % of the MI355X 8 TB/s peak (algorithmic bytes: int4 codes,
  fp16 scales, packed int4 zero points when asymmetric, activations, outputs), the launch plan
  and the measured error against the explicit formula;
* suite ``metadata``: ``recipe`` ("reference" = the reference's input distributions, default;
  "baseline" = the benchmark configuration's), ``zero_point`` ("symmetric" = 8 or "asymmetric",
  baseline recipe only), ``timing_launches``.
"""

from __future__ import annotations

import math
import sys
from statistics import median
from time import perf_counter
from typing import Any, Callable, Literal

from fast_kernels.benchmarking.inputs import algorithmic_bytes, make_case
from fast_kernels.registry import kernel_registry
from fast_kernels.schemas import BenchmarkCase, BenchmarkSuite

WARMUP_ITERS = 4
TIMING_ITERS = 12
DEVICE_TIMING_BLOCKS = 7
WARM_SECONDS = 0.25
CACHE_BUST_BYTES = 2 * 256 * 1024 * 1024
PEAK_HBM_GBS = 8000.0
SubjectKind = Literal["kernel", "baseline"]
VENDOR_BASELINES = ("vendor/cublaslt_fp16_after_dequant", "vendor/hipblaslt_fp16_after_dequant")
REFERENCE_BASELINE = "torch/reference_w4a16_linear"
NATIVE_IMPL = "native"  # kernel impl: the forward over native slabs
_DTYPES = {"fp16": "f16", "bf16": "bf16"}


def _require_torch() -> Any:
    try:
        import torch
    except ImportError:
        return None
    return torch


def _make_case_id(subject_kind: str, subject_id: str, dtype: str, layout: str, shape_name: str) -> str:
    normalized_subject = subject_id.replace("/", "__")
    return f"{subject_kind}-{normalized_subject}-{dtype}-{layout}-{shape_name}"


def _case(subject_kind: SubjectKind, subject_id: str, dtype: str, layout: str, shape_name: str,
          dimensions: dict[str, int], status: str, **fields: Any) -> BenchmarkCase:
    return BenchmarkCase(
        case_id=_make_case_id(subject_kind, subject_id, dtype, layout, shape_name),
        subject_kind=subject_kind,
        subject_id=subject_id,
        dtype=dtype,
        layout=layout,
        shape_name=shape_name,
        dimensions=dimensions,
        status=status,
        **fields,
    )


def _p95(values: list[float]) -> float:
    ordered = sorted(values)
    return ordered[min(len(ordered) - 1, math.ceil(0.95 * len(ordered)) - 1)]


def _time_wall(fn: Callable[[], Any], torch: Any) -> tuple[float, float]:
    """The reference's timing (decode_linear_w4a16.py:131-145): synchronise around every call."""
    torch.cuda.synchronize()
    for _ in range(WARMUP_ITERS):
        fn()
    torch.cuda.synchronize()
    samples: list[float] = []
    for _ in range(TIMING_ITERS):
        torch.cuda.synchronize()
        start = perf_counter()
        fn()
        torch.cuda.synchronize()
        samples.append((perf_counter() - start) * 1e6)
    return float(median(samples)), _p95(samples)


def _time_device(fn: Callable[[int], Any], rotations: int, launches: int, torch: Any) -> tuple[float, float]:
    """Per-launch device time of `launches` back-to-back launches cycling through `rotations`
    weight copies, captured in one HIP graph so host launch overhead does not hide the kernels;
    HIP events between back-to-back graph replays, median and p95 over DEVICE_TIMING_BLOCKS
    replays after at least WARM_SECONDS of warm-up replays."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for r in range(2 * rotations):  # warm-up on the capture stream: workspaces exist before capture
            fn(r % rotations)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(launches):
            fn(i % rotations)
    samples: list[float] = []
    with torch.cuda.stream(stream):
        # Warm for at least WARM_SECONDS of back-to-back replays, so the clocks have ramped
        # after the host-side setup before the first timed block; the blocks then run back to
        # back with no host wait between them.
        first = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        first[0].record(stream)
        graph.replay()
        first[1].record(stream)
        first[1].synchronize()
        block_s = max(first[0].elapsed_time(first[1]) * 1e-3, 1e-6)
        for _ in range(max(DEVICE_TIMING_BLOCKS, min(4096, math.ceil(WARM_SECONDS / block_s)))):
            graph.replay()
        events = [torch.cuda.Event(enable_timing=True) for _ in range(DEVICE_TIMING_BLOCKS + 1)]
        events[0].record(stream)
        for i in range(DEVICE_TIMING_BLOCKS):
            graph.replay()
            events[i + 1].record(stream)
        events[-1].synchronize()
        for i in range(DEVICE_TIMING_BLOCKS):
            samples.append(events[i].elapsed_time(events[i + 1]) * 1e3 / launches)
    del graph
    return float(median(samples)), _p95(samples)


def _upload(torch: Any, case: Any, device: Any) -> tuple[Any, Any, Any, Any]:
    import numpy as np

    act_dtype = torch.float16 if case.act == "f16" else torch.bfloat16
    x = torch.from_numpy(case.x.view(np.int16)).to(device).view(act_dtype)
    q = torch.from_numpy(case.q_u8).to(device)
    a = torch.from_numpy(case.alpha.view(np.int16)).to(device).view(torch.float16)
    b = torch.from_numpy(case.beta.view(np.int16)).to(device).view(torch.float16)
    return x, q, a, b


def _explicit_reference(torch: Any, x: Any, q: Any, a: Any, b: Any, group_size: int) -> Any:
    """fp32 weights alpha*q + beta, fp32 matmul, cast to the activation dtype: the reference's
    explicit formula (decode_linear_w4a16.py:177-192), evaluated on the GPU in row blocks."""
    n = q.shape[0]
    out = torch.empty((x.shape[0], n), device=x.device, dtype=x.dtype)
    x32 = x.float()
    block = max(128, (1 << 27) // max(1, q.shape[1] * 2 * 4))
    for r0 in range(0, n, block):
        r1 = min(n, r0 + block)
        qb = q[r0:r1]
        codes = torch.stack(((qb & 0x0F), (qb >> 4)), dim=-1).reshape(r1 - r0, -1).float()
        scale = a[r0:r1].float().repeat_interleave(group_size, dim=1)
        offset = b[r0:r1].float().repeat_interleave(group_size, dim=1)
        w = codes * scale + offset
        out[:, r0:r1] = (x32 @ w.t()).to(x.dtype)
    return out


def _max_err(actual: Any, expected: Any) -> float:
    return float((actual.float() - expected.float()).abs().max().item())


def _check_close(actual: Any, expected: Any, atol: float, rtol: float, label: str) -> None:
    if tuple(actual.shape) != tuple(expected.shape) or actual.dtype != expected.dtype:
        raise AssertionError(f"{label} shape/dtype mismatch: {tuple(actual.shape)} {actual.dtype} "
                             f"vs {tuple(expected.shape)} {expected.dtype}")
    if bool(actual.float().allclose(expected.float(), atol=atol, rtol=rtol)):
        return
    raise AssertionError(f"{label} mismatch: max_abs_diff={_max_err(actual, expected):.6f}")


def _all_skipped(suite: BenchmarkSuite, reason: str) -> list[BenchmarkCase]:
    cases: list[BenchmarkCase] = []
    for dtype in suite.dtypes:
        for layout in suite.layouts:
            for shape in suite.shapes:
                dims = shape.dimensions()
                for kernel_id in suite.kernels.ids:
                    cases.append(_case("kernel", kernel_id, dtype, layout, shape.name, dims, "skipped",
                                       reason=reason))
                for baseline_id in suite.baselines.ids:
                    cases.append(_case("baseline", baseline_id, dtype, layout, shape.name, dims,
                                       "skipped", reason=reason))
    return cases


def run_decode_linear_w4a16_suite(suite: BenchmarkSuite) -> tuple[list[BenchmarkCase], list[str]]:
    recipe = str(suite.metadata.get("recipe", "reference"))
    asymmetric = recipe == "reference" or suite.metadata.get("zero_point") == "asymmetric"
    launches = int(suite.metadata.get("timing_launches", 100))
    notes = [
        "Runs the W4A16 decode linear on gfx950 HIP kernels when torch-ROCm, a GPU and the native "
        "build are available.",
        f"Wall timing: {WARMUP_ITERS} warmup + {TIMING_ITERS} measured calls with a device "
        "synchronisation around each (the reference's method).",
        f"Device timing: HIP events around a HIP graph of {launches} back-to-back launches, weights rotated through "
        f">= {CACHE_BUST_BYTES >> 20} MiB of copies, median of {DEVICE_TIMING_BLOCKS} blocks.",
        f"Inputs: {recipe} recipe, {'asymmetric' if asymmetric else 'symmetric (zp = 8)'} zero points.",
    ]
    torch = _require_torch()
    if torch is None:
        return _all_skipped(suite, "PyTorch is not installed."), notes
    from fast_kernels.ops import hip_decode_available

    if not hip_decode_available():
        return _all_skipped(suite, "Native module is not built with HIP support."), notes
    if not torch.cuda.is_available():
        return _all_skipped(suite, "torch.cuda.is_available() is false on this machine."), notes
    device = torch.device("cuda")
    props = torch.cuda.get_device_properties(device)
    arch = getattr(props, "gcnArchName", "").split(":")[0]
    notes.append(f"GPU: {torch.cuda.get_device_name(device)} ({arch}, {props.multi_processor_count} CUs, "
                 f"{props.total_memory / 2**30:.0f} GiB)")
    cases: list[BenchmarkCase] = []
    for dtype in suite.dtypes:
        for layout in suite.layouts:
            for shape in suite.shapes:
                print(f"[fk bench] {suite.id}: {dtype} {layout} {shape.name}", file=sys.stderr,
                      flush=True)
                cases.extend(_run_shape(torch, device, suite, dtype, layout, shape, recipe,
                                        asymmetric, launches))
    return cases, notes


def _run_shape(torch: Any, device: Any, suite: BenchmarkSuite, dtype: str, layout: str, shape: Any,
               recipe: str, asymmetric: bool, launches: int) -> list[BenchmarkCase]:
    from fast_kernels.ops import (
        PACKET_FORMATS,
        arc_w4a16_forward,
        arc_w4a16_forward_native,
        arc_w4a16_plan,
        convert_arc_to_native_packets,
        arc_w4a16_supported_impls,
        cublaslt_fp16_after_dequant,
        dequant_w4a16_to_fp16,
        group_size_for_layout,
        pack_arc_w4a16_packets,
    )
    from fast_kernels.ops.decode_quant_linear import KERNEL_AUTO, KERNEL_DOT2, KERNEL_MFMA

    dims = shape.dimensions()
    name = shape.name
    kernels = kernel_registry()
    skip: str | None = None
    group_size = -1
    if dtype not in _DTYPES:
        skip = f"dtype {dtype!r} is not supported (fp16, bf16)"
    else:
        try:
            group_size = group_size_for_layout(layout)
        except ValueError as exc:
            skip = str(exc)
    if skip is None:
        n, k = shape.require_dimension("n"), shape.require_dimension("k")
        if shape.require_dimension("m") != 1:
            skip = "decode suite currently requires shape.m == 1"
        elif n % 128 != 0:
            skip = "decode suite requires n to be divisible by 128"
        elif k % group_size != 0:
            skip = "decode suite requires k to be divisible by group_size"
    if skip is not None:
        return [_case(kind, sid, dtype, layout, name, dims, "skipped", reason=skip)
                for kind, ids in (("baseline", suite.baselines.ids), ("kernel", suite.kernels.ids))
                for sid in ids]

    batch = shape.batch
    act = _DTYPES[dtype]
    atol, rtol = suite.tolerances.atol, suite.tolerances.rtol
    supported = set(arc_w4a16_supported_impls(device)) | {NATIVE_IMPL}
    native_format = "native_asym" if asymmetric else "native_sym"
    out: list[BenchmarkCase] = []
    try:
        case = make_case(batch, n, k, group_size, act=act, asymmetric=asymmetric, recipe=recipe)
        x, q, a, b = _upload(torch, case, device)
        packets = pack_arc_w4a16_packets(q, a, b, group_size=group_size)
        slabs = None
        if any(kernels[kid].impl == NATIVE_IMPL for kid in suite.kernels.ids):
            slabs = convert_arc_to_native_packets(packets, n=n, k=k, group_size=group_size,
                                                  packet_format=native_format)
        explicit = _explicit_reference(torch, x, q, a, b, group_size)
        ref_weight = torch.empty((n, k), device=device, dtype=torch.float16)
        ref_out = torch.empty((batch, n), device=device, dtype=x.dtype)

        def run_reference(qq: Any = q, aa: Any = a, bb: Any = b) -> Any:
            dequant_w4a16_to_fp16(qq, aa, bb, group_size=group_size, output=ref_weight)
            if x.dtype == torch.float16:
                return torch.mm(x, ref_weight.t(), out=ref_out)
            # bf16 activations: the fp16 weights are not representable in bf16, so multiply in fp32
            ref_out.copy_(torch.mm(x.float(), ref_weight.t().float()))
            return ref_out

        run_reference()
        _check_close(ref_out, explicit, atol, rtol, "reference output")
        kernel_out = torch.empty((batch, n), device=device, dtype=x.dtype)
        checked: dict[str, float] = {}
        for kernel_id in suite.kernels.ids:
            impl = kernels[kernel_id].impl
            if impl is not None and (impl not in supported or (impl == "tc" and act != "f16")):
                continue
            if impl == NATIVE_IMPL:
                arc_w4a16_forward_native(x, slabs, n=n, k=k, group_size=group_size,
                                         packet_format=native_format, output=kernel_out)
            else:
                arc_w4a16_forward(x, packets, n=n, k=k, group_size=group_size, output=kernel_out,
                                  impl=impl)
            _check_close(kernel_out, ref_out, atol, rtol, f"{kernel_id} output")
            checked[kernel_id] = _max_err(kernel_out, explicit)
        vendor_out = torch.empty((batch, n), device=device, dtype=torch.float16)
        vendor_weight = torch.empty((n, k), device=device, dtype=torch.float16)
        workspace = torch.empty(8 << 20, device=device, dtype=torch.uint8)
        if act == "f16":
            cublaslt_fp16_after_dequant(x, q, a, b, group_size=group_size, output=vendor_out,
                                        weight_buffer=vendor_weight, workspace=workspace)
            _check_close(vendor_out, ref_out, atol, rtol, "vendor baseline output")
    except Exception as exc:  # noqa: BLE001 - every failure becomes a failed case with its reason
        return [_case(kind, sid, dtype, layout, name, dims, "failed", reason=str(exc))
                for kind, ids in (("baseline", suite.baselines.ids), ("kernel", suite.kernels.ids))
                for sid in ids]

    # Rotated copies so back-to-back launches read HBM, not the Infinity Cache.
    packet_bytes = packets.numel()
    rotations = max(2, math.ceil(CACHE_BUST_BYTES / max(packet_bytes, 1)))
    packet_rot = [packets] + [packets.clone() for _ in range(rotations - 1)]
    slab_rot = [] if slabs is None else [slabs] + [slabs.clone() for _ in range(rotations - 1)]
    qab_rot = [(q, a, b)] + [(q.clone(), a.clone(), b.clone()) for _ in range(rotations - 1)]
    alg_bytes = algorithmic_bytes(batch, n, k, group_size, asymmetric=asymmetric)
    latencies: dict[str, float] = {}

    def timed(kind: SubjectKind, sid: str, wall_fn: Callable[[], Any], dev_fn: Callable[[int], Any],
              extra: dict[str, float]) -> BenchmarkCase:
        wall_med, wall_p95 = _time_wall(wall_fn, torch)
        dev_med, dev_p95 = _time_device(dev_fn, rotations, launches, torch)
        latencies[sid] = dev_med
        metrics = {"hbm_gbs": alg_bytes / dev_med / 1e3,
                   "pct_hbm_peak": 100.0 * alg_bytes / dev_med / 1e3 / PEAK_HBM_GBS,
                   "algorithmic_bytes": float(alg_bytes), **extra}
        return _case(kind, sid, dtype, layout, name, dims, "ok",
                     latency_us_median=dev_med, latency_us_p95=dev_p95,
                     wall_latency_us_median=wall_med, wall_latency_us_p95=wall_p95,
                     device_latency_us_median=dev_med, device_latency_us_p95=dev_p95,
                     throughput=batch * 1e6 / dev_med, decode_tokens_per_second=batch * 1e6 / dev_med,
                     metrics=metrics)

    for kernel_id in suite.kernels.ids:
        impl = kernels[kernel_id].impl
        if impl is not None and impl not in supported:
            out.append(_case("kernel", kernel_id, dtype, layout, name, dims, "skipped",
                             reason=f"{kernel_id} is not supported on "
                                    f"{getattr(torch.cuda.get_device_properties(device), 'gcnArchName', 'this GPU').split(':')[0]}"))
            continue
        if impl == "tc" and act != "f16":
            out.append(_case("kernel", kernel_id, dtype, layout, name, dims, "skipped",
                             reason="the tc (hipBLASLt) path takes fp16 activations only"))
            continue

        if impl == NATIVE_IMPL:
            def run_kernel(p: Any = slabs, impl: str | None = impl) -> Any:
                return arc_w4a16_forward_native(x, p, n=n, k=k, group_size=group_size,
                                                packet_format=native_format, output=kernel_out)
            rot = slab_rot
        else:
            def run_kernel(p: Any = packets, impl: str | None = impl) -> Any:
                return arc_w4a16_forward(x, p, n=n, k=k, group_size=group_size, output=kernel_out,
                                         impl=impl)
            rot = packet_rot

        extra = {"max_abs_err": checked.get(kernel_id, float("nan"))}
        if impl in (None, "scalar", "mfma", NATIVE_IMPL):
            kernel = {"scalar": KERNEL_DOT2, "mfma": KERNEL_MFMA}.get(impl, KERNEL_AUTO)
            plan = arc_w4a16_plan(batch=batch, n=n, k=k, group_size=group_size,
                                  activation_dtype=x.dtype,
                                  packet_format=PACKET_FORMATS[native_format] if impl == NATIVE_IMPL else 0,
                                  kernel=kernel)
            extra.update({f"plan_{key}": float(val) for key, val in plan.items()})
        out.append(timed("kernel", kernel_id, run_kernel, lambda r, f=run_kernel, rot=rot: f(rot[r]), extra))
    # The kernels are timed before the baselines: the reference baseline's large temporaries and
    # long runs measurably slowed the next case timed after them. Cases are reported baselines first.
    kernel_cases = out
    out = []
    vendor_id = next((v for v in suite.baselines.ids if v in VENDOR_BASELINES), None)
    for baseline_id in suite.baselines.ids:
        if baseline_id == REFERENCE_BASELINE:
            out.append(timed("baseline", baseline_id, run_reference,
                             lambda r: run_reference(*qab_rot[r]),
                             {"max_abs_err": _max_err(ref_out, explicit)}))
        elif baseline_id in VENDOR_BASELINES:
            if act != "f16":
                out.append(_case("baseline", baseline_id, dtype, layout, name, dims, "skipped",
                                 reason="the hipBLASLt baseline takes fp16 activations only"))
                continue

            def run_vendor(qq: Any = q, aa: Any = a, bb: Any = b) -> Any:
                return cublaslt_fp16_after_dequant(x, qq, aa, bb, group_size=group_size,
                                                   output=vendor_out, weight_buffer=vendor_weight,
                                                   workspace=workspace)

            out.append(timed("baseline", baseline_id, run_vendor, lambda r: run_vendor(*qab_rot[r]),
                             {"max_abs_err": _max_err(vendor_out, explicit)}))
        else:
            out.append(_case("baseline", baseline_id, dtype, layout, name, dims, "not_implemented",
                             reason=f"{baseline_id} has no runner in this suite family"))

    out.extend(kernel_cases)
    if vendor_id is not None and vendor_id in latencies:
        for c in out:
            if c.status == "ok" and c.subject_id != vendor_id and c.device_latency_us_median:
                c.speedup_vs = {vendor_id: latencies[vendor_id] / c.device_latency_us_median}
    return out


def launch_kernel_case(suite: BenchmarkSuite, case_id: str, launches: int) -> str:
    """Rebuild one kernel case of the suite (the timed run's inputs, packets and rotated weight
    copies) and launch its kernel `launches` times, cycling through the copies, then synchronise.
    For measuring the case under a profiler (``fk bench --counters``); returns the kernel id."""
    import torch

    from fast_kernels.ops import (
        arc_w4a16_forward,
        arc_w4a16_forward_native,
        convert_arc_to_native_packets,
        group_size_for_layout,
        pack_arc_w4a16_packets,
    )

    recipe = str(suite.metadata.get("recipe", "reference"))
    asymmetric = recipe == "reference" or suite.metadata.get("zero_point") == "asymmetric"
    match = [(kid, dtype, layout, shape) for kid in suite.kernels.ids for dtype in suite.dtypes
             for layout in suite.layouts for shape in suite.shapes
             if _make_case_id("kernel", kid, dtype, layout, shape.name) == case_id]
    if not match:
        raise ValueError(f"no kernel case {case_id!r} in suite {suite.id!r}")
    kernel_id, dtype, layout, shape = match[0]
    impl = kernel_registry()[kernel_id].impl
    group_size = group_size_for_layout(layout)
    n, k = shape.require_dimension("n"), shape.require_dimension("k")
    device = torch.device("cuda")
    case = make_case(shape.batch, n, k, group_size, act=_DTYPES[dtype], asymmetric=asymmetric,
                     recipe=recipe)
    x, q, a, b = _upload(torch, case, device)
    packets = pack_arc_w4a16_packets(q, a, b, group_size=group_size)
    native_format = "native_asym" if asymmetric else "native_sym"
    if impl == NATIVE_IMPL:
        packets = convert_arc_to_native_packets(packets, n=n, k=k, group_size=group_size,
                                                packet_format=native_format)
    rotations = max(2, math.ceil(CACHE_BUST_BYTES / max(packets.numel(), 1)))
    copies = [packets] + [packets.clone() for _ in range(rotations - 1)]
    out = torch.empty((shape.batch, n), device=device, dtype=x.dtype)
    for i in range(launches):
        if impl == NATIVE_IMPL:
            arc_w4a16_forward_native(x, copies[i % rotations], n=n, k=k, group_size=group_size,
                                     packet_format=native_format, output=out)
        else:
            arc_w4a16_forward(x, copies[i % rotations], n=n, k=k, group_size=group_size,
                              output=out, impl=impl)
    torch.cuda.synchronize()
    return kernel_id
