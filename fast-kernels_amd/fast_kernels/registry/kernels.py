"""Kernel ids the suites may name (reference: src/fast_kernels/registry/kernels.py:15-136).

The decode/w4a16_linear* ids keep the reference's names, so its suite files verify here; each
maps to an implementation of this package. Ids of the reference's other kernel families are not
registered: suites naming them fail ``fk verify`` with "unknown kernel id".
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class KernelSpec:
    kernel_id: str
    family: str
    description: str
    maturity: str
    impl: str | None = None  # arc_w4a16_forward impl name; None = automatic dispatch;
    # "native" = arc_w4a16_forward_native over slabs converted from the packets


def kernel_registry() -> dict[str, KernelSpec]:
    specs = [
        KernelSpec(
            "decode/w4a16_linear",
            "decode_quant_linear",
            "Automatically dispatched W4A16 decode GEMV over ARC packets (gfx950 HIP).",
            "experimental",
            None,
        ),
        KernelSpec(
            "decode/w4a16_linear_scalar",
            "decode_quant_linear",
            "Stream-K W4A16 GEMV for every batch size: 128-bit packet loads, in-register nibble "
            "dequant, v_dot2 fp32 accumulation, in-kernel activation sums and split-K fix-up "
            "(gfx950 HIP).",
            "experimental",
            "scalar",
        ),
        KernelSpec(
            "decode/w4a16_linear_native",
            "decode_quant_linear",
            "The same GEMV over native gfx950 slabs (slice-major, no fp16 offsets), converted once "
            "from the ARC packets; symmetric or asymmetric slabs follow the case's zero points.",
            "experimental",
            "native",
        ),
        KernelSpec(
            "decode/w4a16_linear_tc",
            "decode_quant_linear",
            "Matrix-core path: packet dequant to fp16, then a hipBLASLt fp16 GEMM.",
            "experimental",
            "tc",
        ),
        KernelSpec(
            "decode/w4a16_linear_mfma",
            "decode_quant_linear",
            "The matrix-core kernel (v_mfma_f32_16x16x32_f16, 16-row m-tiles over 128-column "
            "tiles) for every batch size; no reference counterpart (successor of the tensor-core "
            "ids), timed against decode/w4a16_linear_scalar, the dot2 loop (gfx950 HIP).",
            "experimental",
            "mfma",
        ),
        KernelSpec(
            "decode/w4a16_linear_wgmma",
            "decode_quant_linear",
            "Reference id of a Hopper-only (wgmma) path; skipped on AMD GPUs.",
            "unsupported",
            "wgmma",
        ),
        KernelSpec(
            "template/noop_gemm",
            "gemm",
            "Scaffold-only GEMM entry point for wiring suite definitions.",
            "scaffold",
            None,
        ),
    ]
    return {spec.kernel_id: spec for spec in specs}
