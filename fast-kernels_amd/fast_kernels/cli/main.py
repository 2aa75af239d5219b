"""The ``fk`` command: env, verify, bench, report, plot.

Command names, arguments and exit codes are those of the reference CLI
(src/fast_kernels/cli/main.py:17-117), so its scripts and suite files drive this one; ``bench``
adds ``--counters`` (HBM traffic of every kernel case, measured with rocprofv3). Each command is
one function taking the parsed arguments and returning the exit status; ``COMMANDS`` lists them
with their help text and arguments.
"""

from __future__ import annotations

import argparse
from collections.abc import Callable, Sequence
from pathlib import Path
from typing import NamedTuple


class Option(NamedTuple):
    flags: tuple[str, ...]
    kwargs: dict


class Command(NamedTuple):
    help: str
    options: tuple[Option, ...]
    run: Callable[[argparse.Namespace], int]


def _env(args: argparse.Namespace) -> int:
    from fast_kernels.env import collect_environment

    snapshot = collect_environment()
    if args.json:
        print(snapshot.to_json())
        return 0
    rows = [
        ("python", snapshot.python_version),
        ("platform", snapshot.platform),
        ("machine", snapshot.machine),
        ("git_sha", snapshot.git_sha or "uncommitted"),
        ("git_dirty", snapshot.git_dirty),
        ("torch_version", snapshot.torch_version or "not installed"),
        ("hipcc", snapshot.hipcc_version or "not found"),
        ("cpu_cores", snapshot.cpu_cores),
    ]
    rows += [(f"gpu_{k}", v) for k, v in sorted((snapshot.rocm_smi or {}).items())]
    rows.append(("native_available", snapshot.native.get("available", False)))
    width = max(len(k) for k, _ in rows)
    print("fast-kernels environment")
    for key, value in rows:
        print(f"  {key:<{width}}  {value}")
    return 0


def _verify(args: argparse.Namespace) -> int:
    from fast_kernels.benchmarking import load_suite, verify_suite

    suite = load_suite(args.suite)
    problems = verify_suite(suite)
    if problems:
        print("Suite validation failed:")
        print("\n".join(f"- {p}" for p in problems))
        return 1
    print(f"Suite valid: {suite.id}")
    print(f"{len(suite.kernels.ids)} kernels, {len(suite.baselines.ids)} baselines, "
          f"{len(suite.shapes)} shapes.")
    return 0


def _bench(args: argparse.Namespace) -> int:
    from fast_kernels.benchmarking import benchmark_suite

    run_dir = benchmark_suite(args.suite, args.output_root, counters=args.counters)
    print(f"Wrote benchmark run to {run_dir}")
    return 0


def _report(args: argparse.Namespace) -> int:
    from fast_kernels.reporting import load_result_bundle, render_summary_markdown

    target = Path(args.run_dir) / "summary.md"
    target.write_text(render_summary_markdown(load_result_bundle(args.run_dir)), encoding="utf-8")
    print(f"Updated {target}")
    return 0


def _plot(args: argparse.Namespace) -> int:
    from fast_kernels.reporting import load_result_bundle, render_bandwidth_plot, render_plot

    bundle = load_result_bundle(args.run_dir)
    plots = Path(args.run_dir) / "plots"
    render_plot(bundle, plots / "status_counts.svg")
    render_bandwidth_plot(bundle, plots / "hbm_bandwidth.svg")
    print(f"Updated {plots / 'status_counts.svg'}")
    return 0


_SUITE = Option(("suite",), {"type": Path, "help": "Path to the suite TOML file."})
_RUN_DIR = Option(("run_dir",), {"type": Path, "help": "Path to a run directory."})

COMMANDS: dict[str, Command] = {
    "env": Command("Print environment and build information.",
                   (Option(("--json",), {"action": "store_true",
                                         "help": "Emit JSON instead of a table."}),), _env),
    "verify": Command("Validate a benchmark suite.", (_SUITE,), _verify),
    "bench": Command("Run a benchmark suite and write result artifacts.", (
        _SUITE,
        Option(("--output-root",), {"type": Path, "default": None,
                                    "help": "Override the root directory used for result artifacts."}),
        Option(("--counters",), {"action": "store_true",
                                 "help": "Also measure each kernel case's HBM traffic with rocprofv3 "
                                         "(FETCH_SIZE and WRITE_SIZE, scaled by a copy of known size)."}),
    ), _bench),
    "report": Command("Regenerate summary markdown for a run.", (_RUN_DIR,), _report),
    "plot": Command("Regenerate SVG plots for a run.", (_RUN_DIR,), _plot),
}


def build_parser() -> argparse.ArgumentParser:
    parser = argparse.ArgumentParser(prog="fk", description="fast-kernels (MI355X) development CLI")
    sub = parser.add_subparsers(dest="command", required=True)
    for name, command in COMMANDS.items():
        p = sub.add_parser(name, help=command.help)
        for option in command.options:
            p.add_argument(*option.flags, **option.kwargs)
    return parser


def main(argv: Sequence[str] | None = None) -> int:
    args = build_parser().parse_args(None if argv is None else list(argv))
    return COMMANDS[args.command].run(args)


def entry_point() -> None:
    """Console-script entry (``fk``)."""
    raise SystemExit(main())


if __name__ == "__main__":  # pragma: no cover
    entry_point()


__all__ = ["COMMANDS", "build_parser", "entry_point", "main"]
