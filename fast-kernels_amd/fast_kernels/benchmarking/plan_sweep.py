"""Plan sweep: times every launch plan the library can be steered to at the benchmark shapes, to
check the static dispatch table (plan_w4a16_for_format in arc_w4a16_ops.cpp) against the
alternatives it chooses between.

The reference picks its split-K and kernel per shape by timing candidates on first use
(src/fast_kernels/ops/decode_quant_linear.py:348-380, 442-531, 544-682). This build plans from a
fixed table instead (deterministic, no first-call timing); this sweep is the measurement that
backs the table. Candidates per shape:

  * ``auto``: the table's plan;
  * the plans the table's switches select when one rule is turned off (FK_W4A16_STREAM=0: no
    stream schedule at all; _PIECES, _DIVISOR, _HALF, _HALF_WHOLE, _SMALL = 0: one of its
    fallbacks off; FK_W4A16_STREAM_WPC=2: two workgroups per CU; FK_W4A16_MFMA_STREAM=0: the
    small-batch matrix cores off the stream schedule; FK_W4A16_ARC_QUARTER=0 and
    FK_W4A16_ARC_STREAM=0: the reference packets off the quarter or the whole-tile stream
    schedule);
  * forced K splits (``split_k_slices`` 1, 2, 4, 8: per-slice runs over that many K ranges);
  * for several rows, each kernel choice (dot2 loop, matrix cores).

The switches are read once per process, so each environment runs in a child process of its own.
Every candidate is timed like bench.py's per-shape figure: a HIP graph of >= 200 launches
cycling through rotated weight copies whose total exceeds twice the 256 MiB Infinity Cache,
after 0.3 s of warm-up replays; every plan of a shape is timed in three round-robin passes
(HIP events around one replay, after a warm replay) and its fastest pass is reported.
Candidates with the same plan are timed once.

    python -m fast_kernels.benchmarking.plan_sweep --out ../profiles/plan_sweep.md
"""

from __future__ import annotations

import argparse
import json
import math
import os
import subprocess
import sys
from pathlib import Path
from typing import Any

INFINITY_CACHE_BYTES = 256 * 1024 * 1024

# (config, name, batch, n, k, group_size, activation, packet format): the benchmark configurations'
# shapes (configs[0] is configuration 1's o shape in fp16).
SHAPES: list[tuple[str, str, int, int, int, int, str, str]] = [
    ("1", "7B qkv", 1, 12288, 4096, 128, "f16", "native_sym"),
    ("0/1", "7B o", 1, 4096, 4096, 128, "f16", "native_sym"),
    ("1", "7B gate_up", 1, 22016, 4096, 128, "f16", "native_sym"),
    ("1", "7B down", 1, 4096, 11008, 128, "f16", "native_sym"),
    ("2", "70B qkv", 1, 10240, 8192, 128, "bf16", "native_sym"),
    ("2", "70B o", 1, 8192, 8192, 128, "bf16", "native_sym"),
    ("2", "70B gate_up", 1, 57344, 8192, 128, "bf16", "native_sym"),
    ("2", "70B down", 1, 8192, 28672, 128, "bf16", "native_sym"),
    ("3", "M=2", 2, 14336, 4096, 64, "f16", "native_asym"),
    ("3", "M=4", 4, 14336, 4096, 64, "f16", "native_asym"),
    ("3", "M=8", 8, 14336, 4096, 64, "f16", "native_asym"),
    ("3", "M=16", 16, 14336, 4096, 64, "f16", "native_asym"),
    ("4", "8B qkv", 1, 6144, 4096, 128, "bf16", "native_sym"),
    ("4", "8B o", 1, 4096, 4096, 128, "bf16", "native_sym"),
    ("4", "8B gate_up", 1, 28672, 4096, 128, "bf16", "native_sym"),
    ("4", "8B down", 1, 4096, 14336, 128, "bf16", "native_sym"),
    # the drop-in path: the same shapes over the reference packets
    ("1", "7B qkv arc", 1, 12288, 4096, 128, "f16", "arc"),
    ("0/1", "7B o arc", 1, 4096, 4096, 128, "f16", "arc"),
    ("1", "7B gate_up arc", 1, 22016, 4096, 128, "f16", "arc"),
    ("1", "7B down arc", 1, 4096, 11008, 128, "f16", "arc"),
    ("2", "70B qkv arc", 1, 10240, 8192, 128, "bf16", "arc"),
    ("2", "70B o arc", 1, 8192, 8192, 128, "bf16", "arc"),
    ("2", "70B gate_up arc", 1, 57344, 8192, 128, "bf16", "arc"),
    ("2", "70B down arc", 1, 8192, 28672, 128, "bf16", "arc"),
    ("4", "8B qkv arc", 1, 6144, 4096, 128, "bf16", "arc"),
    ("4", "8B o arc", 1, 4096, 4096, 128, "bf16", "arc"),
    ("4", "8B gate_up arc", 1, 28672, 4096, 128, "bf16", "arc"),
    ("4", "8B down arc", 1, 4096, 14336, 128, "bf16", "arc"),
    ("3", "M=2 arc", 2, 14336, 4096, 64, "f16", "arc"),
    ("3", "M=4 arc", 4, 14336, 4096, 64, "f16", "arc"),
    ("3", "M=8 arc", 8, 14336, 4096, 64, "f16", "arc"),
    ("3", "M=16 arc", 16, 14336, 4096, 64, "f16", "arc"),
    # fewer slices than CUs at 2-16 rows (the reference suite's qkv shape)
    ("-", "4096^2 M=2", 2, 4096, 4096, 64, "f16", "native_asym"),
    ("-", "4096^2 M=16", 16, 4096, 4096, 64, "f16", "native_asym"),
    ("-", "4096^2 M=2 arc", 2, 4096, 4096, 64, "f16", "arc"),
    ("-", "4096^2 M=16 arc", 16, 4096, 4096, 64, "f16", "arc"),
    # long K at 2-8 rows (the reference suite's MLP down shape)
    ("-", "4096x14336 M=2 arc", 2, 4096, 14336, 64, "f16", "arc"),
    ("-", "4096x14336 M=4 arc", 4, 4096, 14336, 64, "f16", "arc"),
    ("-", "4096x14336 M=8 arc", 8, 4096, 14336, 64, "f16", "arc"),
    ("-", "4096x14336 M=4", 4, 4096, 14336, 64, "f16", "native_asym"),
    ("-", "70B qkv M=4 arc", 4, 10240, 8192, 128, "bf16", "arc"),
    ("-", "70B down M=4 arc", 4, 8192, 28672, 128, "bf16", "arc"),
    ("-", "70B down M=8", 8, 8192, 28672, 128, "bf16", "native_sym"),
    # one row at G = 64 (the reference suite's shapes)
    ("-", "14336x4096 G64 arc", 1, 14336, 4096, 64, "f16", "arc"),
    ("-", "14336x4096 G64", 1, 14336, 4096, 64, "f16", "native_asym"),
    ("-", "4096x14336 G64 arc", 1, 4096, 14336, 64, "f16", "arc"),
    ("-", "4096^2 G64 arc", 1, 4096, 4096, 64, "f16", "arc"),
    # a divisor grid or pieces (896 slices, K/G = 64)
    ("-", "28672x8192 arc", 1, 28672, 8192, 128, "bf16", "arc"),
    ("-", "28672x8192", 1, 28672, 8192, 128, "bf16", "native_sym"),
]
# the reference's own suite (benchmarks/suites/decode_linear_w4a16.toml): its shapes over the
# reference packets at 1-8 rows, both group sizes, fp16
SHAPES += [
    ("suite", f"ref {n}x{k} G{g} M={m}", m, n, k, g, "f16", "arc")
    for g in (64, 128)
    for n, k in ((4096, 4096), (14336, 4096), (4096, 14336))
    for m in (1, 2, 4, 8)
]

# Environments (one child process each): name -> variables.
ENVS: dict[str, dict[str, str]] = {
    "auto": {},
    "no_stream": {"FK_W4A16_STREAM": "0"},
    "no_pieces": {"FK_W4A16_STREAM_PIECES": "0"},
    "no_divisor": {"FK_W4A16_STREAM_DIVISOR": "0"},
    "no_half": {"FK_W4A16_STREAM_HALF": "0"},
    "no_half_whole": {"FK_W4A16_HALF_WHOLE": "0"},
    "no_small": {"FK_W4A16_STREAM_SMALL": "0"},
    "wpc2": {"FK_W4A16_STREAM_WPC": "2"},
    "no_mfma_stream": {"FK_W4A16_MFMA_STREAM": "0"},
    "no_arc_quarter": {"FK_W4A16_ARC_QUARTER": "0"},
    "no_arc_stream": {"FK_W4A16_ARC_STREAM": "0"},
    "no_arc_eighths": {"FK_W4A16_ARC_EIGHTHS": "0"},
    "no_arc_mfma_stream": {"FK_W4A16_ARC_MFMA_STREAM": "0"},
}
SPLITS = (1, 2, 3, 4, 6, 8, 16)
KERNELS = {"auto": 0, "dot2": 1, "mfma": 2}
FORMATS = {"arc": 0, "native_sym": 1, "native_asym": 2}
PLAN_KEYS = ("m_tile", "workgroups", "groups_per_workgroup", "slice_cols", "schedule")
SCHEDULE_NAMES = {0: "runs", 1: "pairs", 2: "stream"}


def _plan_label(plan: dict[str, int]) -> str:
    s = SCHEDULE_NAMES.get(plan.get("schedule", 0), "?")
    return (f"{s} wg={plan['workgroups']} gpw={plan['groups_per_workgroup']} "
            f"cols={plan['slice_cols']} mt={plan['m_tile']}")


def _plan_id(plan: dict[str, int]) -> tuple[int, ...]:
    return tuple(int(plan[k]) for k in PLAN_KEYS)


class _Shape:
    """Rotated weight copies of one shape on the GPU (seeded, reference recipe: codes U{0..15},
    scales U[0.001, 0.02], zp = 8 or U{0..15}), converted to the shape's packet format."""

    def __init__(self, torch: Any, native: Any, batch: int, n: int, k: int, g: int, act: str,
                 fmt: str) -> None:
        from fast_kernels.ops import arc_packet_stride_bytes, packet_stride_bytes

        self.batch, self.n, self.k, self.g = batch, n, k, g
        self.act_code = 1 if act == "bf16" else 0
        self.fmt = FORMATS[fmt]
        dtype = torch.bfloat16 if act == "bf16" else torch.float16
        dev = torch.device("cuda")
        gen = torch.Generator(device=dev)
        gen.manual_seed((batch * 1_000_003 + n * 1009 + k * 101 + g) % (2**31 - 1))
        ng = k // g
        stride = arc_packet_stride_bytes(g)
        weight_bytes = n * k // 2 + n * ng * 4
        rotations = max(2, math.ceil(2 * INFINITY_CACHE_BYTES / weight_bytes) + 1)
        stream = torch.cuda.current_stream().cuda_stream
        self.packets = []
        native_fmt = self.fmt != FORMATS["arc"]
        rows, row_bytes = (((n // 32) * ng, packet_stride_bytes(g, fmt)) if native_fmt
                           else ((n // 128) * ng, stride))
        # every copy in one allocation, as bench.py places them
        pool = torch.empty((rotations, rows, row_bytes), device=dev, dtype=torch.uint8)
        for r in range(rotations):
            q = torch.randint(0, 256, (n, k // 2), device=dev, dtype=torch.uint8, generator=gen)
            alpha = (0.001 + 0.019 * torch.rand((n, ng), device=dev, generator=gen)).to(torch.float16)
            if self.fmt == FORMATS["native_asym"]:
                zp = torch.randint(0, 16, (n, ng), device=dev, generator=gen).to(torch.float16)
                beta = -(alpha * zp)
            else:
                beta = -(alpha * 8)
            pk = (torch.empty(((n // 128) * ng, stride), device=dev, dtype=torch.uint8)
                  if native_fmt else pool[r])
            native.pack_arc_w4a16_packets(q.data_ptr(), alpha.data_ptr(), beta.data_ptr(),
                                          pk.data_ptr(), n, k, g, stride, stream)
            if native_fmt:
                arc = pk
                pk = pool[r]
                native.convert_arc_to_native_packets(arc.data_ptr(), pk.data_ptr(), n, k, g,
                                                     self.fmt, stream)
                del arc
            self.packets.append(pk)
            del q, alpha, beta
        self.x = torch.randn((batch, k), device=dev, generator=gen).to(dtype)
        self.out = torch.empty((batch, n), device=dev, dtype=dtype)


def _candidate_runner(torch: Any, native: Any, shp: _Shape, split: int, kernel: int,
                      launches: int) -> tuple[Any, int]:
    """A captured graph of >= `launches` launches of one candidate over the rotated copies, and
    its launch count."""
    plan = dict(native.arc_w4a16_plan(shp.batch, shp.n, shp.k, shp.g, shp.act_code, split, 0,
                                      shp.fmt, kernel))
    ws = torch.zeros(max(1, plan["workspace_bytes"]) + 256, device="cuda", dtype=torch.uint8)
    R = len(shp.packets)
    reps = max(1, -(-launches // R))

    def fn() -> None:
        stream = torch.cuda.current_stream().cuda_stream
        for _ in range(reps):
            for r in range(R):
                native.w4a16_forward_kernel(
                    shp.x.data_ptr(), shp.packets[r].data_ptr(), shp.out.data_ptr(),
                    ws.data_ptr(), ws.numel(), shp.batch, shp.n, shp.k, shp.g, shp.fmt,
                    shp.act_code, split, kernel, stream)

    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        fn()
    graph.ws = ws  # keep the workspace alive with the graph
    graph.side = side
    return graph, reps * R


def _time_graph(torch: Any, graph: Any, count: int) -> float:
    """Microseconds per launch over one replay (HIP events on the graph's stream), after one
    warm replay."""
    side = graph.side
    with torch.cuda.stream(side):
        graph.replay()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(side)
        graph.replay()
        end.record(side)
        end.synchronize()
    return start.elapsed_time(end) * 1e3 / count


def child(env_name: str, launches: int, only: list[str], auto_plans: dict[str, list[int]]) -> int:
    """Runs in a child process with the environment already set: prints one JSON line per
    (shape, plan). Candidates with the same plan are timed once (their names joined); plans equal
    to the automatic one (auto_plans, from the "auto" process) are skipped. Every plan is timed in
    three round-robin passes over the shape's plans, after 0.3 s of warm-up replays, and its
    fastest pass is reported (the first plan timed would otherwise pay for the clocks ramping)."""
    import time

    import torch

    from fast_kernels.native import native_module

    native = native_module()
    for config, name, batch, n, k, g, act, fmt in SHAPES:
        if only and name not in only:
            continue
        act_code = 1 if act == "bf16" else 0
        cands: list[tuple[str, int, int]] = [(env_name, 0, 0)]
        if env_name == "auto":
            cands += [(f"split_k={s}", s, 0) for s in SPLITS if s <= k // g]
            if batch > 1:
                cands += [(f"kernel={kn}", 0, kv) for kn, kv in KERNELS.items() if kv]
        plans: dict[tuple[int, ...], dict[str, Any]] = {}
        for label, split, kernel in cands:
            try:
                plan = dict(native.arc_w4a16_plan(batch, n, k, g, act_code, split, 0,
                                                  FORMATS[fmt], kernel))
            except Exception as exc:  # a candidate the table cannot build for this shape
                print(json.dumps({"shape": name, "cand": label, "error": str(exc)}), flush=True)
                continue
            pid = _plan_id(plan)
            if env_name != "auto" and list(pid) == auto_plans.get(name):
                continue  # the automatic plan, timed by the "auto" process
            if pid in plans:
                plans[pid]["names"].append(label)
            else:
                plans[pid] = {"names": [label], "split": split, "kernel": kernel, "plan": plan}
        if not plans:
            continue
        shp = _Shape(torch, native, batch, n, k, g, act, fmt)
        runners = {pid: _candidate_runner(torch, native, shp, c["split"], c["kernel"], launches)
                   for pid, c in plans.items()}
        first = next(iter(runners.values()))
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < 0.3:
            _time_graph(torch, *first)
        best: dict[tuple[int, ...], float] = {}
        for _ in range(3):
            for pid, (graph, count) in runners.items():
                us = _time_graph(torch, graph, count)
                best[pid] = min(best.get(pid, us), us)
        for pid, c in plans.items():
            print(json.dumps({"config": config, "shape": name, "cand": c["names"][0],
                              "names": c["names"], "us": round(best[pid], 3),
                              "plan": {k2: int(c["plan"][k2]) for k2 in PLAN_KEYS},
                              "bytes": n * k // 2 + n * (k // g) * 2 +
                              (n * (k // g) // 2 if fmt == "native_asym" else 0) +
                              batch * k * 2 + batch * n * 2}), flush=True)
        del runners, first, shp
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return 0


def _markdown(rows: list[dict[str, Any]], command: str) -> str:
    by_shape: dict[str, list[dict[str, Any]]] = {}
    for r in rows:
        if "us" in r:
            by_shape.setdefault(r["shape"], []).append(r)
    lines = [
        "# Plan sweep: the static dispatch table against its alternatives",
        "",
        f"Command: `{command}`",
        "",
        "Each candidate is timed as bench.py times a shape (a HIP graph of >= 200 launches over",
        "rotated weight copies beyond twice the Infinity Cache; every plan of a shape timed in",
        "three round-robin passes, the fastest kept). Candidates with the same plan are listed",
        "together. `auto/best` is the automatic plan's time over the fastest plan's.",
        "",
        "| config | shape | auto plan | auto us | best candidate | best us | auto/best |",
        "|---|---|---|---:|---|---:|---:|",
    ]
    detail = ["", "## Every candidate", ""]
    for config, name, *_ in SHAPES:
        cands = by_shape.get(name)
        if not cands:
            continue
        auto = next((c for c in cands if c["cand"] == "auto"), None)
        if auto is None:
            continue
        uniq: dict[tuple[int, ...], dict[str, Any]] = {}
        for c in cands:
            pid = _plan_id(c["plan"])
            names = list(c.get("names", [c["cand"]]))
            if pid not in uniq or c["us"] < uniq[pid]["us"]:
                names = uniq[pid]["names"] + names if pid in uniq else names
                uniq[pid] = dict(c, names=names)
            else:
                uniq[pid]["names"].extend(names)
        auto_us = uniq[_plan_id(auto["plan"])]["us"]
        best = min(uniq.values(), key=lambda c: c["us"])
        ratio = auto_us / best["us"]
        lines.append(f"| {config} | {name} | {_plan_label(auto['plan'])} | {auto_us:.2f} | "
                     f"{', '.join(best['names'][:3])} | {best['us']:.2f} | {ratio:.3f} |")
        detail.append(f"### {name}")
        detail.append("")
        detail.append("| candidates (same plan) | plan | us | GB/s |")
        detail.append("|---|---|---:|---:|")
        for c in sorted(uniq.values(), key=lambda c: c["us"]):
            detail.append(f"| {', '.join(c['names'])} | {_plan_label(c['plan'])} | {c['us']:.2f} "
                          f"| {c['bytes'] / (c['us'] * 1e-6) / 1e9:.0f} |")
        detail.append("")
    return "\n".join(lines + detail) + "\n"


def main(argv: list[str] | None = None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--out", default="", help="markdown report path (JSON rows beside it)")
    p.add_argument("--launches", type=int, default=200)
    p.add_argument("--envs", default=",".join(ENVS), help="comma list of environments")
    p.add_argument("--only", default="", help="comma list of shape names")
    p.add_argument("--child", default="", help=argparse.SUPPRESS)
    p.add_argument("--auto-plans", default="{}", help=argparse.SUPPRESS)
    args = p.parse_args(argv)
    only = [s for s in args.only.split(",") if s]
    if args.child:
        return child(args.child, args.launches, only, json.loads(args.auto_plans))
    rows: list[dict[str, Any]] = []
    for env_name in [e for e in args.envs.split(",") if e]:
        env = dict(os.environ, **ENVS[env_name])
        auto_plans = {r["shape"]: list(_plan_id(r["plan"])) for r in rows
                      if r.get("cand") == "auto" and "plan" in r}
        cmd = [sys.executable, "-m", "fast_kernels.benchmarking.plan_sweep", "--child", env_name,
               "--launches", str(args.launches), "--auto-plans", json.dumps(auto_plans)]
        if only:
            cmd += ["--only", ",".join(only)]
        print(f"[plan_sweep] {env_name}", flush=True)
        # the child's lines are echoed as they come (a long sweep shows its progress)
        proc = subprocess.Popen(cmd, env=env, stdout=subprocess.PIPE, text=True,
                                cwd=str(Path(__file__).resolve().parents[2]))
        assert proc.stdout is not None
        for line in proc.stdout:
            print(line.rstrip(), flush=True)
            if line.startswith("{"):
                rows.append(json.loads(line))
        if proc.wait(timeout=900) != 0:
            return proc.returncode
    command = "python -m fast_kernels.benchmarking.plan_sweep " + " ".join(
        a for a in (argv if argv is not None else sys.argv[1:]))
    report = _markdown(rows, command.strip())
    if args.out:
        Path(args.out).write_text(report)
        Path(args.out).with_suffix(".json").write_text(json.dumps(rows, indent=0))
    print(report)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
