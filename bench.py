"""Benchmark: W4A16 GEMV effective HBM bandwidth on one MI355X (the headline metric).

Workload (benchmark configuration 2): one Llama-70B-class layer's four M=1 decode projections,
group size 128, symmetric int4 (zp = 8), bf16 activations and outputs:
    qkv 10240x8192, o 8192x8192, gate_up 57344x8192, down 8192x28672.
A "step" is one pass over the four GEMVs. Weights are random int4 codes (synthetic, seeded on the
device), packed into the reference packet layout and, for the headline (--packets native_sym, the
default), converted on the GPU to the native symmetric slabs: the same code words (8 codes along K
per uint32, the reference's packing) and alphas, laid out slice-major for contiguous streaming,
without the fp16 offsets that zp = 8 fixes. The other format (--packets arc: the reference packets
as the drop-in entry points take them) is measured too, in a child process, and reported under
"other_packets". Shape b has R_b rotated weight copies (together more than twice the 256 MiB
Infinity Cache), step s uses copy s mod R_b of it, and R_b is chosen so that a graph's restart at
copy 0 does not bring a copy back early, so every launch streams its weights from HBM.

Timing: exactly K steps, launched as one replay of a HIP graph of K steps (torch.cuda.CUDAGraph;
step s uses weight copy s mod R_b of shape b) between HIP events on the capture stream. The
warm-up replays that same graph (ceil(W / K) times, so at least W untimed steps), since the first
replay of a freshly instantiated graph runs about 1 % slower. The warm-up is enqueued after a
synchronisation and the start event right behind it, so the host enqueues the timed replay while
the GPU runs the warm-up and the timed interval holds no host launch latency. (--graph chunked
instead replays a W-step graph K // W times plus a graph of the K mod W left-over steps; a
replay boundary every W steps measured up to 1 us per step slower at W = 5.) The graphs are
captured before the per-shape runs below, which keep the GPU busy up to the warm-up (after an
idle capture a replay runs slower for its first tens of milliseconds while the clocks ramp up).
value = algorithmic bytes
per step / time per step (int4 codes + fp16 scales + activations + outputs; the reference
packets' fp16 beta, when measured, is read but not credited).

Also reported: per-shape us/call and GB/s (each shape's own graph of >= 300 launches, replayed once),
a roofline object for the dominant kernel (gate_up), and the reference's CPU arithmetic (fp32
accumulation) timed on all of this process's host cores on a bounded sample of the workload.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO_ROOT / "fast-kernels_amd"))
sys.path.insert(0, str(REPO_ROOT))

PEAK_HBM_GBS = 8000.0
INFINITY_CACHE_BYTES = 256 * 1024 * 1024

WORKLOADS = {
    # name: (activation dtype, group size, [(shape name, N, K)])
    "llama70b_layer_m1_bf16": (
        "bf16",
        128,
        [("qkv", 10240, 8192), ("o", 8192, 8192), ("gate_up", 57344, 8192), ("down", 8192, 28672)],
    ),
    "llama8b_layer_m1_bf16": (
        "bf16",
        128,
        [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 28672, 4096), ("down", 4096, 14336)],
    ),
    "llama7b_layer_m1_fp16": (
        "f16",
        128,
        [("qkv", 12288, 4096), ("o", 4096, 4096), ("gate_up", 22016, 4096), ("down", 4096, 11008)],
    ),
}


# Launch schedules of a plan (fk_arc_w4a16_plan.schedule) and the kernel each runs.
SCHEDULES = {0: "runs", 1: "slice_pairs", 2: "stream"}


def kernel_name(packets: str, schedule: int) -> str:
    if packets == "arc":
        return "w4a16_gemv_kernel"
    return "w4a16_gemv_stream_kernel" if schedule == 2 else "w4a16_gemv_native_kernel"


def algorithmic_bytes(batch: int, n: int, k: int, g: int) -> int:
    return n * k // 2 + n * (k // g) * 2 + batch * k * 2 + batch * n * 2


def _threads_per_workgroup(plan: dict, num_groups: int) -> int:
    """Threads of one workgroup: 256 for the per-slice runs, 8 waves for the stream schedule and a
    ninth (the control wave) when its workgroups also take a piece of a left-over slice."""
    if plan.get("schedule", 0) != 2:
        return 256
    return 576 if plan["groups_per_workgroup"] % num_groups else 512


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1000)  # 1000 steps of the 70B layer: 80 ms
    p.add_argument("--warmup", type=int, default=200)
    p.add_argument(
        "--graph",
        choices=["single", "chunked"],
        default="single",
        help="single: the K timed steps are one replay of a K-step graph, warmed by replaying it; "
        "chunked: replays of a W-step graph (a replay boundary every W steps)",
    )
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="llama70b_layer_m1_bf16")
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--split-k", type=int, default=0, help="0 = built-in plan")
    p.add_argument("--only", default="", help="comma list of shape names to run (profiling)")
    p.add_argument("--per-shape-launches", type=int, default=300)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--eager", action="store_true", help="launch without a HIP graph")
    p.add_argument(
        "--packets",
        choices=["arc", "native_sym"],
        default="native_sym",
        help="packet format of the headline value: the native symmetric slabs (default) or the "
        "reference packets (arc)",
    )
    p.add_argument(
        "--no-other-packets",
        action="store_true",
        help="skip measuring the other packet format (reported under 'other_packets')",
    )
    p.add_argument(
        "--copy-calibration",
        action="store_true",
        help="only run a plain 256 MiB device-to-device copy 10 times (scales rocprofv3 "
        "FETCH_SIZE / WRITE_SIZE to bytes)",
    )
    return p.parse_args()


COPY_CALIBRATION_BYTES = 256 * 1024 * 1024


def copy_calibration(torch) -> int:
    src = torch.empty(COPY_CALIBRATION_BYTES, device="cuda", dtype=torch.uint8).random_(0, 255)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": COPY_CALIBRATION_BYTES, "launches": 10}))
    return 0


class ShapeBuffers:
    def __init__(self, torch, native, name, n, k, g, batch, act, rotations, split_k, packets="arc"):
        from fast_kernels.ops import PACKET_FORMATS, arc_packet_stride_bytes, packet_stride_bytes

        self.name, self.n, self.k, self.g, self.batch = name, n, k, g, batch
        self.stride = arc_packet_stride_bytes(g)
        self.format = PACKET_FORMATS[packets]
        self.native_stride = packet_stride_bytes(g, packets)
        self.act_code = 1 if act == "bf16" else 0
        dtype = torch.bfloat16 if act == "bf16" else torch.float16
        dev = torch.device("cuda")
        gen = torch.Generator(device=dev)
        gen.manual_seed((batch * 1_000_003 + n * 1009 + k * 101 + g) % (2**31 - 1))
        self.packets = []
        ng = k // g
        native_fmt = self.format != PACKET_FORMATS["arc"]
        rows, row_bytes = (((n // 32) * ng, self.native_stride) if native_fmt
                           else ((n // 128) * ng, self.stride))
        # All copies of the shape's weights in one allocation, as a loader would place a model's
        # weights (measured on MI355X, alternating runs: the 70B step 72.3-72.5 -> 71.8-72.0 us
        # against one allocation per copy between the generator's temporaries).
        pool = torch.empty((rotations, rows, row_bytes), device=dev, dtype=torch.uint8)
        for r in range(rotations):
            q = torch.randint(0, 256, (n, k // 2), device=dev, dtype=torch.uint8, generator=gen)
            alpha = (0.001 + 0.019 * torch.rand((n, ng), device=dev, generator=gen)).to(torch.float16)
            beta = -(alpha * 8)
            pk = (torch.empty(((n // 128) * ng, self.stride), device=dev, dtype=torch.uint8)
                  if native_fmt else pool[r])
            native.pack_arc_w4a16_packets(
                q.data_ptr(), alpha.data_ptr(), beta.data_ptr(), pk.data_ptr(), n, k, g,
                self.stride, torch.cuda.current_stream().cuda_stream,
            )
            if native_fmt:
                arc = pk
                pk = pool[r]
                native.convert_arc_to_native_packets(
                    arc.data_ptr(), pk.data_ptr(), n, k, g, self.format,
                    torch.cuda.current_stream().cuda_stream,
                )
                del arc
            self.packets.append(pk)
            del q, alpha, beta
        self.x = torch.randn((batch, k), device=dev, generator=gen).to(dtype)
        self.out = torch.empty((batch, n), device=dev, dtype=dtype)
        self.plan = dict(
            native.arc_w4a16_plan(batch, n, k, g, self.act_code, split_k, 0, self.format)
        )
        self.split_k = split_k
        self.bytes = algorithmic_bytes(batch, n, k, g)

    def launch(self, native, torch, ws, r):
        stream = torch.cuda.current_stream().cuda_stream
        pk = self.packets[r % len(self.packets)].data_ptr()
        if self.format == 0:
            native.arc_w4a16_forward_ex(
                self.x.data_ptr(), pk, self.out.data_ptr(), ws.data_ptr(), ws.numel(), self.batch,
                self.n, self.k, self.g, self.stride, self.act_code, self.split_k, stream,
            )
        else:
            native.arc_w4a16_forward_native(
                self.x.data_ptr(), pk, self.out.data_ptr(), ws.data_ptr(), ws.numel(), self.batch,
                self.n, self.k, self.g, self.format, self.act_code, self.split_k, stream,
            )


def rotations_for(total_packet_bytes: int) -> int:
    return max(2, math.ceil(2 * INFINITY_CACHE_BYTES / max(1, total_packet_bytes)) + 1)


def step_rotations(chunk: int, r_min: int, min_chunk: int) -> int:
    """Weight copies of every shape in the step graphs: at least r_min (each shape's own count,
    so that R copies of any one shape exceed twice the Infinity Cache), and chosen so that the
    copy sequence also stays cold where a graph of `chunk` steps starts over at copy 0: step s of
    a graph uses copy s mod R of every shape, so copy 0 comes back after chunk mod R steps at a
    replay boundary. That is 0 (a seamless cycle), or at least min_chunk steps (more than twice
    the Infinity Cache of step traffic), or the graph is shorter than R."""
    r = max(1, r_min)
    while not (chunk <= r or chunk % r == 0 or chunk % r >= min_chunk):
        r += 1
    return r


def step_chunk(steps: int, warmup: int, min_chunk: int) -> tuple[int, bool]:
    """Steps per graph of the timed run and whether the warm-up is that graph's first replay:
    W steps per graph when W spans at least min_chunk steps (a graph restarts at weight copy 0)
    and is shorter than the run, else one graph of all K steps with a warm-up graph of its own.
    The timed run is steps // chunk replays plus a graph of steps % chunk: exactly K steps."""
    use = min_chunk <= warmup < steps
    return (warmup if use else steps), use


def make_runner(torch, fn, launches_per_call: int, eager: bool):
    """Returns run(times) that issues `times` x launches_per_call launches on the current stream."""
    if eager:
        def run(times):
            for _ in range(times):
                fn()
        return run
    graph = torch.cuda.CUDAGraph()
    fn()  # warm (first call may size the workspace cache; nothing allocates under capture)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        fn()
    torch.cuda.synchronize()

    def run(times):
        for _ in range(times):
            graph.replay()
    return run


def time_events(torch, run, reps: int, lead=None) -> float:
    """Milliseconds for run(reps), by HIP events on the current stream.

    lead: untimed work enqueued after the synchronisation and before the start event (the
    warm-up). While the GPU runs it, the host enqueues the timed launches, so the timed interval
    starts with the GPU busy instead of waiting for the host's first graph launch (tens of
    microseconds, which a short timed run of 20 steps would otherwise count as 1-2 %)."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    if lead is not None:
        lead()
    start.record()
    run(reps)
    end.record()
    end.synchronize()
    return float(start.elapsed_time(end))


def measured_traffic(workload: str, shape: str, packets: str = "native_sym"):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 PMC summary
    (profiles/w4a16_gemv_traffic.json, FETCH_SIZE + WRITE_SIZE scaled by a plain copy of known
    size), or None when no measurement for this workload and shape is committed."""
    path = REPO_ROOT / "profiles" / "w4a16_gemv_traffic.json"
    if not path.exists():
        return None
    try:
        data = json.loads(path.read_text())
        entry = data[packets][workload][shape]
        return int(entry["hbm_bytes_per_launch"])
    except (KeyError, ValueError, TypeError):
        return None


def cpu_baseline(workload: str, batch: int, seconds: float) -> dict:
    """The reference's CPU arithmetic (fp32 weights alpha*q + beta, fp32 accumulation, one cast:
    decode_linear_w4a16.py:177-192 restated in oracle/w4a16_oracle.c fko_gemv_f32) on the same
    shapes, host-generated inputs, OpenMP over every core this process may run on, timed over
    whole passes of the four shapes until at least `seconds` have passed."""
    from fast_kernels.benchmarking.inputs import make_case
    from oracle import oracle

    act, g, shapes = WORKLOADS[workload]
    threads = len(os.sched_getaffinity(0))
    oracle.set_threads(threads)
    cases = [make_case(batch, n, k, g, act=act) for _, n, k in shapes]
    total_bytes = 0
    t0 = time.perf_counter()
    passes = 0
    while True:
        for c in cases:
            oracle.gemv_f32(c.x, c.q_u8, c.alpha, c.beta, g, act)
            total_bytes += algorithmic_bytes(batch, c.n, c.k, g)
        passes += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds:
            break
    return {
        "value": round(total_bytes / elapsed / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{passes} full pass(es) over the {len(shapes)} {workload} GEMVs "
        f"({elapsed:.1f} s, oracle/w4a16_oracle.c fko_gemv_f32: fp32 weights and fp32 "
        f"accumulation as the reference computes them, OpenMP {threads} threads)",
    }


def measure(torch, native, args, act, g, shapes, packets):
    """Per-shape and whole-step timing over packets of one format. The buffers are freed before
    returning except for what the report needs (plans, byte counts)."""
    # Shape b has R_b weight copies and step s uses copy s mod R_b of it. R_b is the fewest
    # copies whose total exceeds twice the Infinity Cache, raised where needed so that a graph's
    # restart at copy 0 does not bring a copy back early (step_rotations). The weights of all
    # copies stay few (a larger footprint adds TLB misses that a minimal rotation does not have).
    step_bytes = sum(algorithmic_bytes(args.batch, n, k, g) for _, n, k in shapes)
    min_chunk = rotations_for(step_bytes)
    if args.graph == "single":
        chunk, use_chunks = args.steps, False
    else:
        chunk, use_chunks = step_chunk(args.steps, args.warmup, min_chunk)
    bufs = []
    for name, n, k in shapes:
        pk_bytes = (n // 128) * (k // g) * (128 * g // 2 + 512)
        r_b = step_rotations(chunk, rotations_for(pk_bytes), min_chunk)
        bufs.append(
            ShapeBuffers(torch, native, name, n, k, g, args.batch, act, r_b, args.split_k,
                         packets)
        )
    ws_bytes = max(max(b.plan["workspace_bytes"] for b in bufs), 1)
    ws = torch.zeros(ws_bytes + 256, device="cuda", dtype=torch.uint8)
    torch.cuda.synchronize()
    # Whole step: step s of a graph launches every shape with rotation s mod R, so consecutive
    # steps read different weight copies.

    def steps_fn(count):
        def fn():
            for s_i in range(count):
                for b in bufs:
                    b.launch(native, torch, ws, s_i)
        return fn

    # Steady state: the K timed steps are one replay of a K-step graph (--graph single), or
    # replays of a W-step graph plus a graph of the K mod W left-over steps (--graph chunked).
    # Either way the timed replays are not a graph's first (about 1 % slower, 0.8 us per 70B step
    # on MI355X). A graph's steps start over at copy 0; the copy counts above keep that cold.
    run_chunk = make_runner(torch, steps_fn(chunk), chunk * len(bufs), args.eager)
    left = args.steps % chunk
    run_left = make_runner(torch, steps_fn(left), left * len(bufs), args.eager) if left else None
    if args.graph == "single":
        # The warm-up replays the timed graph itself (ceil(W / K) times, so at least W steps):
        # the timed replay is then not the graph's first, which runs about 1 % slower.
        reps_warm = -(-args.warmup // args.steps) if args.warmup > 0 else 0
        warm = (lambda times, r=reps_warm: run_chunk(times * r)) if reps_warm else None
    elif use_chunks:
        warm = run_chunk
    else:  # no warm-up, or one too short to chunk the run or of at least K steps: its own graph
        warm = (make_runner(torch, steps_fn(args.warmup), args.warmup * len(bufs), args.eager)
                if args.warmup > 0 else None)

    def run_steps(times):
        for _ in range(times):
            run_chunk(args.steps // chunk)
            if run_left is not None:
                run_left(1)

    # Per-shape timing: each shape's own graph of reps x R launches (its R rotations in turn),
    # replayed once between events, so that no graph launch boundary falls inside the run.
    per_shape = {}
    for b in bufs:
        R = len(b.packets)
        reps = max(1, -(-args.per_shape_launches // R))

        def shape_fn(b=b, R=R, reps=reps):
            for _ in range(reps):
                for r in range(R):
                    b.launch(native, torch, ws, r)

        run = make_runner(torch, shape_fn, reps * R, args.eager)
        # warm as long as the timed run: the first shape otherwise pays for the clocks ramping up
        time_events(torch, run, 1)
        ms = time_events(torch, run, 1)
        us = ms * 1e3 / (reps * R)
        per_shape[b.name] = {
            "n": b.n,
            "k": b.k,
            "us_per_call": round(us, 3),
            "gbs": round(b.bytes / (us * 1e-6) / 1e9, 1),
            "pct_peak": round(100.0 * b.bytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 1),
            "bytes": b.bytes,
            "rotations": R,
            "groups_per_workgroup": b.plan["groups_per_workgroup"],
            "workgroups": b.plan["workgroups"],
            "slice_cols": b.plan["slice_cols"],
            "schedule": SCHEDULES[b.plan.get("schedule", 0)],
            "threads_per_workgroup": _threads_per_workgroup(b.plan, b.k // b.g),
        }

    # The step's graphs were captured before the per-shape runs, so the GPU has been streaming
    # right up to the warm-up: the capture of thousands of launches leaves it idle long enough
    # for its clocks to drop, and a replay right after idle runs slower for its first tens of ms.
    # The warm-up replay leads the timed replays with no synchronisation in between, so the
    # host enqueues the timed graphs while the GPU runs the warm-up.
    ms = time_events(torch, run_steps, 1, lead=(lambda: warm(1)) if warm is not None else None)
    torch.cuda.synchronize()
    steps = args.steps
    ms_per_step = ms / steps
    step_bytes = sum(b.bytes for b in bufs)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9

    for b in bufs:
        b.packets = [None] * len(b.packets)
    del ws
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return bufs, per_shape, value, ms_per_step, steps


def measure_other_packets(args) -> dict:
    """The same step over the other packet format, measured by this script in a child process.

    A second measurement in the same process, after the first one's buffers are freed, ran its
    per-shape graphs up to 2 us slower at gate_up (both formats, either order, on MI355X; the
    step graph much less), so each format gets a fresh process. The parent holds no buffers
    meanwhile."""
    other_format = "native_sym" if args.packets == "arc" else "arc"
    cmd = [sys.executable, str(Path(__file__).resolve()), "--packets", other_format,
           "--no-other-packets", "--no-cpu-baseline", "--steps", str(args.steps), "--warmup",
           str(args.warmup), "--graph", args.graph, "--workload", args.workload, "--batch",
           str(args.batch), "--split-k", str(args.split_k), "--per-shape-launches",
           str(args.per_shape_launches)]
    if args.only:
        cmd += ["--only", args.only]
    if args.eager:
        cmd.append("--eager")
    proc = subprocess.run(cmd, capture_output=True, text=True, timeout=900, check=False)
    if proc.returncode != 0:
        raise RuntimeError(f"other-packets measurement failed ({proc.returncode}): "
                           f"{proc.stderr[-2000:]}")
    line = [ln for ln in proc.stdout.splitlines() if ln.startswith("{")][-1]
    child = json.loads(line)
    return {"packets": other_format, "value": child["value"],
            "ms_per_step": child["ms_per_step"], "per_shape": child["per_shape"]}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py measures one GPU only: this build has no multi-GPU path (asked for "
            f"--gpus {args.gpus}). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    import torch

    from fast_kernels.native import native_module

    native = native_module()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    if args.copy_calibration:
        return copy_calibration(torch)
    act, g, shapes = WORKLOADS[args.workload]
    if args.only:
        keep = set(args.only.split(","))
        shapes = [s for s in shapes if s[0] in keep]

    first = measure(torch, native, args, act, g, shapes, args.packets)
    other = None
    if not args.no_other_packets:
        other = measure_other_packets(args)
    bufs, per_shape, value, ms_per_step, steps = first

    dominant = max(bufs, key=lambda b: b.bytes)
    dom = per_shape[dominant.name]
    achieved = dom["gbs"]
    result = {
        "metric": "W4A16 GEMV effective HBM GB/s (% of MI355X peak) + us/call, M=1",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": act if act == "bf16" else "fp16",
        "data": "synthetic (seeded random int4 codes, fp16 scales U[0.001,0.02], zp=8, x~N(0,1))",
        "config": {
            "workload": args.workload,
            "batch": args.batch,
            "group_size": g,
            "shapes": {b.name: [b.n, b.k] for b in bufs},
            "step": "one pass over the listed GEMVs, launched from a HIP graph",
            "cache_busting": "rotated weight copies > 2 x 256 MiB per shape",
            "packets": args.packets,
        },
        "pct_peak": round(100.0 * value / PEAK_HBM_GBS, 1),
        "per_shape": per_shape,
        "roofline": {
            "bound": "hbm",
            "kernel": kernel_name(args.packets, dominant.plan.get("schedule", 0))
            + f" ({dominant.name} {dominant.n}x{dominant.k})",
            "achieved": achieved,
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": measured_traffic(args.workload, dominant.name, args.packets),
        },
    }
    if other is not None:
        result["other_packets"] = {
            "packets": other["packets"],
            "value": other["value"],
            "unit": "GB/s",
            "ms_per_step": other["ms_per_step"],
            "pct_peak": round(100.0 * other["value"] / PEAK_HBM_GBS, 1),
            "per_shape_us": {k: v["us_per_call"] for k, v in other["per_shape"].items()},
            "note": "same step and algorithmic bytes over the other packet format, measured in a "
            "child process",
        }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.workload, args.batch, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
