"""Suite verification and execution (reference: src/fast_kernels/benchmarking/runner.py:19-156).

``verify_suite`` applies the reference's checks (known kernel and baseline ids, non-empty shapes,
dtypes and layouts). ``benchmark_suite`` runs a suite's family runner and writes the result
bundle under ``<output_root>/<suite id>/<UTC time>-<git sha>/``. Suites of families without a
runner here produce not_implemented cases, as the reference does for scaffold suites.
"""

from __future__ import annotations

from collections import Counter
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


def _make_case_id(subject_kind: str, subject_id: str, dtype: str, layout: str, shape_name: str) -> str:
    return f"{subject_kind}-{subject_id.replace('/', '__')}-{dtype}-{layout}-{shape_name}"


def verify_suite(suite: BenchmarkSuite) -> list[str]:
    errors: list[str] = []
    kernels = kernel_registry()
    baselines = baseline_registry()
    if not suite.kernels.ids:
        errors.append("suite defines no kernels")
    if not suite.baselines.ids:
        errors.append("suite defines no baselines")
    errors += [f"unknown kernel id: {kid}" for kid in suite.kernels.ids if kid not in kernels]
    errors += [f"unknown baseline id: {bid}" for bid in suite.baselines.ids if bid not in baselines]
    if not suite.shapes:
        errors.append("suite defines no shapes")
    if not suite.dtypes:
        errors.append("suite defines no dtypes")
    if not suite.layouts:
        errors.append("suite defines no layouts")
    return errors


def _scaffold_cases(suite: BenchmarkSuite) -> list[BenchmarkCase]:
    cases: list[BenchmarkCase] = []
    for kind, ids in (("kernel", suite.kernels.ids), ("baseline", suite.baselines.ids)):
        for subject_id in ids:
            for dtype in suite.dtypes:
                for layout in suite.layouts:
                    for shape in suite.shapes:
                        cases.append(
                            BenchmarkCase(
                                case_id=_make_case_id(kind, subject_id, dtype, layout, shape.name),
                                subject_kind=kind,
                                subject_id=subject_id,
                                dtype=dtype,
                                layout=layout,
                                shape_name=shape.name,
                                dimensions=shape.dimensions(),
                                status="not_implemented",
                                reason=f"{subject_id} is registered but scaffold-only.",
                            )
                        )
    return cases


def _execute_suite(suite: BenchmarkSuite) -> tuple[list[BenchmarkCase], list[str]]:
    if suite.family == "decode_quant_linear":
        return run_decode_linear_w4a16_suite(suite)
    if suite.family == "decode_step_w4a16":
        return run_decode_step_w4a16_suite(suite)
    return _scaffold_cases(suite), [
        f"Scaffold run: no runner for suite family {suite.family!r}.",
        "Result artifacts validate the suite, registry and reporting flow.",
    ]


def benchmark_suite(suite_path: str | Path, output_root: str | Path | None = None) -> Path:
    suite = load_suite(suite_path)
    errors = verify_suite(suite)
    if errors:
        raise ValueError("Suite validation failed:\n" + "\n".join(f"- {e}" for e in errors))
    repo = repo_root()
    env = collect_environment(repo)
    created_at = datetime.now(tz=timezone.utc)
    run_id = f"{created_at.strftime('%Y%m%dT%H%M%SZ')}-{env.git_sha or 'worktree'}"
    cases, notes = _execute_suite(suite)
    metadata = RunMetadata(
        run_id=run_id,
        suite_id=suite.id,
        created_at=created_at.isoformat(),
        git_sha=env.git_sha,
        python_version=env.python_version,
        platform=env.platform,
        machine=env.machine,
        native=env.native,
        torch_version=env.torch_version,
        rocm_smi=env.rocm_smi,
        hipcc_version=env.hipcc_version,
        cpu_cores=env.cpu_cores,
        notes=notes,
    )
    bundle = ResultBundle(metadata=metadata, cases=cases)
    root = Path(output_root) if output_root is not None else default_results_root()
    run_dir = root / suite.id / run_id
    write_result_bundle(run_dir, bundle)
    return run_dir


def summarize_statuses(bundle: ResultBundle) -> dict[str, int]:
    return dict(Counter(case.status for case in bundle.cases))
