"""fk bench on the GPU: small suites of both runner families must produce only ok/skipped cases,
with the gates (kernel vs reference baseline vs explicit fp32 formula) passing."""

from __future__ import annotations

from pathlib import Path

import pytest

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

from fast_kernels.benchmarking import benchmark_suite  # noqa: E402
from fast_kernels.reporting import load_result_bundle  # noqa: E402

LINEAR = """
schema_version = 1
id = "tiny_decode_linear"
family = "decode_quant_linear"
description = "tiny"
dtypes = ["fp16", "bf16"]
layouts = ["groupwise_64", "groupwise_128"]
[kernels]
ids = ["decode/w4a16_linear", "decode/w4a16_linear_scalar", "decode/w4a16_linear_tc", "decode/w4a16_linear_wgmma"]
[baselines]
ids = ["torch/reference_w4a16_linear", "vendor/hipblaslt_fp16_after_dequant"]
[tolerances]
atol = 0.0625
rtol = 0.01
[metadata]
recipe = "{recipe}"
timing_launches = 20
[[shapes]]
name = "s1"
m = 1
n = 1024
k = 2048
batch = 1
[[shapes]]
name = "s4"
m = 1
n = 512
k = 1024
batch = 4
"""

STEP = """
schema_version = 1
id = "tiny_decode_step"
family = "decode_step_w4a16"
description = "tiny"
dtypes = ["bf16"]
layouts = ["groupwise_128"]
[kernels]
ids = ["decode/w4a16_linear"]
[baselines]
ids = ["torch/reference_w4a16_linear"]
[tolerances]
atol = 0.0625
rtol = 0.01
[metadata]
layers = 3
[[shapes]]
name = "qkv"
m = 1
n = 768
k = 512
[[shapes]]
name = "down"
m = 1
n = 512
k = 1792
"""


@pytest.mark.parametrize("recipe", ["reference", "baseline"])
def test_decode_linear_suite_runs(tmp_path: Path, recipe: str) -> None:
    suite = tmp_path / "tiny.toml"
    suite.write_text(LINEAR.replace("{recipe}", recipe))
    bundle = load_result_bundle(benchmark_suite(suite, output_root=tmp_path))
    statuses = {c.case_id: c.status for c in bundle.cases}
    assert "failed" not in statuses.values(), [c.reason for c in bundle.cases if c.status == "failed"]
    ok = [c for c in bundle.cases if c.status == "ok"]
    # per (layout, shape): fp16 -> auto, scalar, tc, reference, vendor; bf16 -> auto, scalar, reference
    assert len(ok) == 2 * 2 * (5 + 3)
    for c in ok:
        assert c.device_latency_us_median > 0 and c.metrics["hbm_gbs"] > 0
    wgmma = [c for c in bundle.cases if c.subject_id.endswith("_wgmma")]
    assert wgmma and all(c.status == "skipped" for c in wgmma)
    auto = [c for c in ok if c.subject_id == "decode/w4a16_linear" and c.dtype == "fp16"]
    assert auto and all("vendor/hipblaslt_fp16_after_dequant" in c.speedup_vs for c in auto)


def test_decode_step_suite_runs(tmp_path: Path) -> None:
    suite = tmp_path / "step.toml"
    suite.write_text(STEP)
    bundle = load_result_bundle(benchmark_suite(suite, output_root=tmp_path))
    assert all(c.status == "ok" for c in bundle.cases), [c.reason for c in bundle.cases]
    step = [c for c in bundle.cases if c.shape_name == "decode_step" and c.subject_kind == "kernel"]
    assert len(step) == 1 and step[0].metrics["hbm_gbs"] > 0
    assert "torch/reference_w4a16_linear" in step[0].speedup_vs
