"""Result-bundle schema written by ``fk bench`` (metadata.json, results.json, results.csv).

Keeps the reference's field names and schema_version 2 (src/fast_kernels/schemas/results.py:8-51)
so result bundles from either build load with either reporter. Additions: the ROCm environment
(``rocm_smi``, ``hipcc_version``) in the run metadata; per-case device timing, HBM figures and
the launch plan go into ``metrics``.
"""

from __future__ import annotations

from typing import Any, Literal

from pydantic import BaseModel, Field


class RunMetadata(BaseModel):
    schema_version: int = 2
    run_id: str
    suite_id: str
    created_at: str
    git_sha: str | None = None
    python_version: str
    platform: str
    machine: str
    native: dict[str, Any] = Field(default_factory=dict)
    nvidia_smi: dict[str, str] | None = None
    nvcc_version: str | None = None
    torch_version: str | None = None
    rocm_smi: dict[str, str] | None = None
    hipcc_version: str | None = None
    cpu_cores: int | None = None
    notes: list[str] = Field(default_factory=list)


class BenchmarkCase(BaseModel):
    case_id: str
    subject_kind: Literal["kernel", "baseline"]
    subject_id: str
    dtype: str
    layout: str
    shape_name: str
    dimensions: dict[str, int]
    status: Literal["ok", "skipped", "not_implemented", "failed"]
    latency_us_median: float | None = None
    latency_us_p95: float | None = None
    wall_latency_us_median: float | None = None
    wall_latency_us_p95: float | None = None
    device_latency_us_median: float | None = None
    device_latency_us_p95: float | None = None
    throughput: float | None = None
    decode_tokens_per_second: float | None = None
    context_tokens_per_second: float | None = None
    effective_kv_gib_per_second: float | None = None
    speedup_vs: dict[str, float] = Field(default_factory=dict)
    metrics: dict[str, float] = Field(default_factory=dict)
    reason: str | None = None


class ResultBundle(BaseModel):
    schema_version: int = 2
    metadata: RunMetadata
    cases: list[BenchmarkCase] = Field(default_factory=list)
