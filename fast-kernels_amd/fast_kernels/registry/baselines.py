"""Baseline ids the suites may name (reference: src/fast_kernels/registry/baselines.py:14-88)."""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class BaselineSpec:
    baseline_id: str
    source: str
    description: str
    maturity: str


def baseline_registry() -> dict[str, BaselineSpec]:
    specs = [
        BaselineSpec(
            "torch/reference_w4a16_linear",
            "framework",
            "Dequantize to fp16 (native kernel) plus torch.mm.",
            "experimental",
        ),
        BaselineSpec(
            "vendor/hipblaslt_fp16_after_dequant",
            "vendor",
            "hipBLASLt fp16 GEMM after native W4A16 dequantization.",
            "experimental",
        ),
        BaselineSpec(
            "vendor/cublaslt_fp16_after_dequant",
            "vendor",
            "Reference id of the vendor baseline; served by hipBLASLt on AMD GPUs.",
            "experimental",
        ),
        BaselineSpec(
            "torch/reference_gemm",
            "framework",
            "PyTorch reference GEMM baseline placeholder.",
            "scaffold",
        ),
        BaselineSpec(
            "vendor/hipblaslt_gemm",
            "vendor",
            "hipBLASLt GEMM baseline placeholder.",
            "scaffold",
        ),
        BaselineSpec(
            "vendor/cublaslt_gemm",
            "vendor",
            "Reference id of the vendor GEMM placeholder.",
            "scaffold",
        ),
    ]
    return {spec.baseline_id: spec for spec in specs}
