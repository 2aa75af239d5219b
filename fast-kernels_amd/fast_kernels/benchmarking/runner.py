"""Suite checks and suite runs behind ``fk verify`` and ``fk bench``.

The checks and the bundle location are the interface the reference defines
(src/fast_kernels/benchmarking/runner.py:19-156): a suite is valid when it names at least one
kernel and one baseline, every id is registered, and it has shapes, dtypes and layouts; a run
writes ``<output root>/<suite id>/<UTC timestamp>-<git sha>/``. The rest is this package's own:

* the family runners are looked up in ``FAMILY_RUNNERS``; a suite of a family with no runner here
  (the reference's other kernel families, template suites) yields one ``not_implemented`` case per
  (subject, dtype, layout, shape), so its bundle still validates the registry-to-report flow;
* ``counters=True`` measures each kernel case's HBM traffic with rocprofv3 after the timed run
  (``fast_kernels.benchmarking.counters``) and adds it to the case metrics.
"""

from __future__ import annotations

import itertools
from collections import Counter
from collections.abc import Callable
from datetime import datetime, timezone
from pathlib import Path

from fast_kernels.benchmarking.decode_linear_w4a16 import run_decode_linear_w4a16_suite
from fast_kernels.benchmarking.decode_step_w4a16 import run_decode_step_w4a16_suite
from fast_kernels.benchmarking.suites import load_suite
from fast_kernels.env import collect_environment
from fast_kernels.paths import default_results_root, repo_root
from fast_kernels.registry import baseline_registry, kernel_registry
from fast_kernels.reporting.artifacts import write_result_bundle
from fast_kernels.schemas import BenchmarkCase, BenchmarkSuite, ResultBundle, RunMetadata

FamilyRunner = Callable[[BenchmarkSuite], "tuple[list[BenchmarkCase], list[str]]"]

FAMILY_RUNNERS: dict[str, FamilyRunner] = {
    "decode_quant_linear": run_decode_linear_w4a16_suite,
    "decode_step_w4a16": run_decode_step_w4a16_suite,
}


def verify_suite(suite: BenchmarkSuite) -> list[str]:
    """Every problem with the suite, in a fixed order (empty list: valid)."""
    known_kernels, known_baselines = kernel_registry(), baseline_registry()
    problems = []
    for label, ids in (("kernels", suite.kernels.ids), ("baselines", suite.baselines.ids)):
        if not ids:
            problems.append(f"suite defines no {label}")
    problems += [f"unknown kernel id: {i}" for i in suite.kernels.ids if i not in known_kernels]
    problems += [f"unknown baseline id: {i}" for i in suite.baselines.ids if i not in known_baselines]
    for label, values in (("shapes", suite.shapes), ("dtypes", suite.dtypes),
                          ("layouts", suite.layouts)):
        if not values:
            problems.append(f"suite defines no {label}")
    return problems


def _placeholder_cases(suite: BenchmarkSuite) -> list[BenchmarkCase]:
    subjects = [("kernel", i) for i in suite.kernels.ids] + [("baseline", i) for i in suite.baselines.ids]
    cases = []
    for (kind, sid), dtype, layout, shape in itertools.product(
            subjects, suite.dtypes, suite.layouts, suite.shapes):
        case_id = "-".join((kind, sid.replace("/", "__"), dtype, layout, shape.name))
        cases.append(BenchmarkCase(
            case_id=case_id, subject_kind=kind, subject_id=sid, dtype=dtype, layout=layout,
            shape_name=shape.name, dimensions=shape.dimensions(), status="not_implemented",
            reason=f"{sid} is registered but scaffold-only."))
    return cases


def run_cases(suite: BenchmarkSuite) -> tuple[list[BenchmarkCase], list[str]]:
    """The suite's cases and run notes from its family runner (or placeholders)."""
    runner = FAMILY_RUNNERS.get(suite.family)
    if runner is not None:
        return runner(suite)
    return _placeholder_cases(suite), [
        f"Scaffold run: no runner for suite family {suite.family!r}.",
        "Result artifacts validate the suite, registry and reporting flow.",
    ]


def benchmark_suite(suite_path: str | Path, output_root: str | Path | None = None,
                    counters: bool = False) -> Path:
    """Run a suite and write its result bundle; returns the run directory."""
    suite = load_suite(suite_path)
    problems = verify_suite(suite)
    if problems:
        raise ValueError("Suite validation failed:\n" + "\n".join(f"- {p}" for p in problems))
    env = collect_environment(repo_root())
    started = datetime.now(tz=timezone.utc)
    run_id = f"{started:%Y%m%dT%H%M%SZ}-{env.git_sha or 'worktree'}"
    cases, notes = run_cases(suite)
    if counters:
        from fast_kernels.benchmarking.counters import add_traffic_metrics

        notes = notes + add_traffic_metrics(Path(suite_path), cases)
    metadata = RunMetadata(
        run_id=run_id, suite_id=suite.id, created_at=started.isoformat(), git_sha=env.git_sha,
        python_version=env.python_version, platform=env.platform, machine=env.machine,
        native=env.native, torch_version=env.torch_version, rocm_smi=env.rocm_smi,
        hipcc_version=env.hipcc_version, cpu_cores=env.cpu_cores, notes=notes)
    run_dir = Path(output_root or default_results_root()) / suite.id / run_id
    write_result_bundle(run_dir, ResultBundle(metadata=metadata, cases=cases))
    return run_dir


def summarize_statuses(bundle: ResultBundle) -> dict[str, int]:
    return dict(Counter(case.status for case in bundle.cases))
