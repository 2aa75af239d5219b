"""The fk harness on the CPU: CLI commands, suite files, registry, runners' skip path and the
result-bundle round trip (mirrors the reference's tests/python/test_cli.py, test_suites.py,
test_decode_benchmark.py and tests/reporting/test_artifacts.py)."""

from __future__ import annotations

import json
from pathlib import Path

import pytest

from fast_kernels.benchmarking import benchmark_suite, load_suite, verify_suite
from fast_kernels.cli.main import main
from fast_kernels.registry import baseline_registry, kernel_registry
from fast_kernels.reporting import load_result_bundle
from fast_kernels.reporting.artifacts import write_result_bundle
from fast_kernels.schemas import BenchmarkCase, ResultBundle, RunMetadata

SUITES = Path("benchmarks/suites")
BASELINE_SUITES = {
    "w4a16_cpu_reference_shape.toml": (["fp16"], ["groupwise_128"], 1),
    "w4a16_llama7b_m1.toml": (["fp16"], ["groupwise_128"], 4),
    "w4a16_llama70b_m1.toml": (["bf16"], ["groupwise_128"], 4),
    "w4a16_smallbatch_g64_asym.toml": (["fp16"], ["groupwise_64"], 4),
    "w4a16_llama8b_decode_step.toml": (["bf16"], ["groupwise_128"], 4),
}


def test_env_command_json(capsys: pytest.CaptureFixture[str]) -> None:
    assert main(["env", "--json"]) == 0
    payload = json.loads(capsys.readouterr().out)
    assert "python_version" in payload and "native" in payload
    assert payload["native"]["available"] is True
    assert payload["native"]["compiled_with_hip"] is True
    assert payload["cpu_cores"] >= 1


def test_env_command_table() -> None:
    assert main(["env"]) == 0


def test_every_suite_verifies() -> None:
    files = sorted(SUITES.glob("*.toml"))
    assert len(files) >= 7
    for path in files:
        suite = load_suite(path)
        assert verify_suite(suite) == [], path
        assert main(["verify", str(path)]) == 0


def test_reference_decode_suite_shape_matrix() -> None:
    suite = load_suite(SUITES / "decode_linear_w4a16.toml")
    assert suite.id == "decode_linear_w4a16"
    assert suite.kernels.ids == [
        "decode/w4a16_linear",
        "decode/w4a16_linear_scalar",
        "decode/w4a16_linear_tc",
        "decode/w4a16_linear_wgmma",
    ]
    assert "torch/reference_w4a16_linear" in suite.baselines.ids
    assert suite.layouts == ["groupwise_64", "groupwise_128"]
    assert len(suite.shapes) == 12
    assert suite.tolerances.atol == 0.0625 and suite.tolerances.rtol == 0.01


@pytest.mark.parametrize("name", sorted(BASELINE_SUITES))
def test_baseline_config_suites(name: str) -> None:
    dtypes, layouts, n_shapes = BASELINE_SUITES[name]
    suite = load_suite(SUITES / name)
    assert suite.dtypes == dtypes and suite.layouts == layouts and len(suite.shapes) == n_shapes


def test_registry_keeps_reference_ids() -> None:
    kernels = kernel_registry()
    for kid in ("decode/w4a16_linear", "decode/w4a16_linear_scalar", "decode/w4a16_linear_tc",
                "decode/w4a16_linear_wgmma"):
        assert kid in kernels
    baselines = baseline_registry()
    assert "vendor/cublaslt_fp16_after_dequant" in baselines
    assert "vendor/hipblaslt_fp16_after_dequant" in baselines


def test_verify_reports_unknown_ids(tmp_path: Path) -> None:
    text = (SUITES / "template_gemm.toml").read_text()
    bad = tmp_path / "bad.toml"
    bad.write_text(text.replace("template/noop_gemm", "decode/clustered_page_decode_auto"))
    errors = verify_suite(load_suite(bad))
    assert errors == ["unknown kernel id: decode/clustered_page_decode_auto"]
    assert main(["verify", str(bad)]) == 1


def test_bench_command_writes_artifacts(tmp_path: Path) -> None:
    assert main(["bench", str(SUITES / "template_gemm.toml"), "--output-root", str(tmp_path)]) == 0
    run_dirs = list((tmp_path / "template_gemm").iterdir())
    assert len(run_dirs) == 1
    run_dir = run_dirs[0]
    for rel in ("metadata.json", "results.json", "results.csv", "summary.md", "plots/status_counts.svg"):
        assert (run_dir / rel).exists(), rel
    bundle = load_result_bundle(run_dir)
    assert {c.status for c in bundle.cases} == {"not_implemented"}
    assert main(["report", str(run_dir)]) == 0
    assert main(["plot", str(run_dir)]) == 0
    assert (run_dir / "plots" / "status_counts.svg").read_text().startswith("<svg")


@pytest.mark.parametrize("name", ["decode_linear_w4a16.toml", "w4a16_llama8b_decode_step.toml"])
def test_decode_suites_write_artifacts_when_skipped(tmp_path: Path, name: str) -> None:
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("exercises the no-GPU path")
    run_dir = benchmark_suite(SUITES / name, output_root=tmp_path)
    bundle = load_result_bundle(run_dir)
    assert bundle.cases
    assert {c.status for c in bundle.cases} == {"skipped"}
    assert all(c.reason for c in bundle.cases)
    assert (run_dir / "summary.md").exists()
    assert bundle.metadata.cpu_cores and bundle.metadata.hipcc_version


def test_result_bundle_round_trip(tmp_path: Path) -> None:
    bundle = ResultBundle(
        metadata=RunMetadata(run_id="test-run", suite_id="demo", created_at="2026-04-14T00:00:00+00:00",
                             python_version="3.10.12", platform="linux", machine="x86_64",
                             native={"available": True}, notes=["demo"]),
        cases=[BenchmarkCase(case_id="kernel-demo-fp16-row_major-shape0", subject_kind="kernel",
                             subject_id="template/noop_gemm", dtype="fp16", layout="row_major",
                             shape_name="shape0", dimensions={"m": 1, "n": 2, "k": 3, "batch": 1},
                             status="ok", device_latency_us_median=2.0,
                             metrics={"hbm_gbs": 1000.0, "pct_hbm_peak": 12.5})],
    )
    write_result_bundle(tmp_path, bundle)
    loaded = load_result_bundle(tmp_path)
    assert loaded == bundle
    assert loaded.schema_version == 2 and loaded.metadata.schema_version == 2
    assert (tmp_path / "plots" / "hbm_bandwidth.svg").exists()
    assert "1000.0" in (tmp_path / "summary.md").read_text()


def test_plan_sweep_report_groups_same_plans_and_ratios() -> None:
    """The plan sweep's report (fast_kernels.benchmarking.plan_sweep): candidates with the same
    plan are listed together, and auto/best compares the automatic plan with the fastest one."""
    from fast_kernels.benchmarking.plan_sweep import _markdown

    plan_a = {"m_tile": 1, "workgroups": 256, "groups_per_workgroup": 64, "slice_cols": 32,
              "schedule": 2}
    plan_b = dict(plan_a, schedule=0)
    rows = [
        {"config": "2", "shape": "70B o", "cand": "auto", "names": ["auto", "split_k=1"],
         "us": 7.5, "plan": plan_a, "bytes": 34635776},
        {"config": "2", "shape": "70B o", "cand": "no_stream", "names": ["no_stream"],
         "us": 7.0, "plan": plan_b, "bytes": 34635776},
    ]
    md = _markdown(rows, "cmd")
    assert "| 2 | 70B o | stream wg=256 gpw=64 cols=32 mt=1 | 7.50 | no_stream | 7.00 | 1.071 |" in md
    assert "| auto, split_k=1 | stream" in md
