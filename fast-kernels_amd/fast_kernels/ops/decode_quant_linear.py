"""Python op API of the W4A16 decode linear ("ARC") path on MI355X.

Mirrors the reference module (src/fast_kernels/ops/decode_quant_linear.py): same public names,
keyword arguments, tensor checks, error types and environment override. What runs underneath is
the gfx950 library (libfk_w4a16.so) through ``fast_kernels._native``; nothing here computes on the
CPU, and every op raises RuntimeError when the extension is missing.

Differences from the reference, by design:
  * impl "auto" dispatches by batch on the HIP kernels (dot2 loop below 8 rows, matrix cores from
    8); "scalar" is the dot2 (FMA) loop for every batch and "mfma" (no reference counterpart) the
    matrix-core kernel for every batch, so the suites can time the two against each other.
  * impl "scalar" is one HIP launch (in-kernel activation sums and split-K fix-up) instead of a
    group-sum prepass plus a GEMV plus an optional reduction; "auto" picks it by a static rule
    rather than timing candidates on the first call (decode_quant_linear.py:442-682), so results
    and launch choices do not depend on timing noise.
  * impl "tc" (reference: dequant + cuBLASLt) is dequant + hipBLASLt; "wgmma" (Hopper only in the
    reference) is not offered on gfx950.
  * activations may be bf16 as well as fp16 (output in the same dtype) on the "scalar" impl.
"""

from __future__ import annotations

import os
from typing import TYPE_CHECKING, Any

from fast_kernels.native import native_build_info, native_module

if TYPE_CHECKING:  # pragma: no cover
    import torch

_ARC_WORKSPACE_CACHE: dict[tuple[int, int], Any] = {}
_ARC_SPLIT_K_PARTIALS_CACHE: dict[tuple[int, int, int, int], Any] = {}
_ARC_WEIGHT_BUFFER_CACHE: dict[tuple[int, int, int], Any] = {}
_ARC_VENDOR_WORKSPACE_CACHE: dict[tuple[int, int], Any] = {}

_ARC_IMPL_ENV = "FK_ARC_W4A16_IMPL"
_ARC_IMPL_AUTO = "auto"
_ARC_IMPL_SCALAR = "scalar"
_ARC_IMPL_TC = "tc"
_ARC_IMPL_WGMMA = "wgmma"
_ARC_IMPL_MFMA = "mfma"
_ARC_IMPLS = {_ARC_IMPL_AUTO, _ARC_IMPL_SCALAR, _ARC_IMPL_TC, _ARC_IMPL_WGMMA, _ARC_IMPL_MFMA}
# Kernel choice of the HIP GEMV per impl (FK_KERNEL_* in include/fk_w4a16.h): "auto" dispatches
# by batch (dot2 loop below 8 rows, matrix cores from 8), "scalar" is the dot2 (FMA) loop for every
# batch, "mfma" the matrix-core kernel for every batch.
KERNEL_AUTO, KERNEL_DOT2, KERNEL_MFMA = 0, 1, 2
_IMPL_KERNEL = {_ARC_IMPL_AUTO: KERNEL_AUTO, _ARC_IMPL_SCALAR: KERNEL_DOT2,
                _ARC_IMPL_MFMA: KERNEL_MFMA}
_VENDOR_WORKSPACE_BYTES = 32 * 1024 * 1024

ACT_F16 = 0
ACT_BF16 = 1

LAYOUT_TO_GROUP_SIZE: dict[str, int] = {
    "groupwise_64": 64,
    "groupwise_128": 128,
}


def _require_torch() -> Any:
    try:
        import torch
    except ImportError as exc:  # pragma: no cover
        raise RuntimeError("PyTorch is required for decode_quant_linear ops") from exc
    return torch


def hip_decode_available() -> bool:
    info = native_build_info()
    return bool(info.get("available", False)) and bool(info.get("compiled_with_hip", False))


def cuda_decode_available() -> bool:
    """Reference name (decode_quant_linear.py:47-49): true when the GPU backend is built."""
    return hip_decode_available()


def group_size_for_layout(layout: str) -> int:
    try:
        return LAYOUT_TO_GROUP_SIZE[layout]
    except KeyError as exc:
        raise ValueError(f"unsupported layout: {layout}") from exc


def arc_packet_stride_bytes(group_size: int) -> int:
    """Bytes per packet: 128 columns x G/2 code bytes + 128 fp16 alpha + 128 fp16 beta."""
    if group_size not in {64, 128}:
        raise ValueError("group_size must be 64 or 128")
    return (128 * (group_size // 2)) + (2 * 128 * 2)


def _require_gpu_backend() -> Any:
    native = native_module()
    if not hip_decode_available():
        raise RuntimeError("fast-kernels native module was built without HIP support")
    return native


def _check_gpu_tensor(tensor: Any, *, name: str, dtype: Any, ndim: int) -> None:
    torch = _require_torch()
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    dtypes = dtype if isinstance(dtype, tuple) else (dtype,)
    if tensor.dtype not in dtypes:
        raise TypeError(f"{name} must have dtype {' or '.join(str(d) for d in dtypes)}")
    if tensor.ndim != ndim:
        raise ValueError(f"{name} must be {ndim}D")
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_same_device(*named_tensors: tuple[str, Any]) -> None:
    devices = {tensor.device for _, tensor in named_tensors}
    if len(devices) <= 1:
        return
    summary = ", ".join(f"{name}={tensor.device}" for name, tensor in named_tensors)
    raise ValueError(f"all GPU tensors must be on the same device: {summary}")


def _current_stream_ptr(device: Any) -> int:
    torch = _require_torch()
    return int(torch.cuda.current_stream(device=device).cuda_stream)


def _device_index(device: Any) -> int:
    return int(device.index or 0)


def arc_w4a16_supported_impls(device: Any | None = None) -> tuple[str, ...]:
    """Implementations available on this build: auto, scalar (HIP dot2 GEMV), mfma (HIP
    matrix-core kernel) and tc (hipBLASLt)."""
    impls = [_ARC_IMPL_AUTO, _ARC_IMPL_SCALAR, _ARC_IMPL_MFMA]
    if hip_decode_available():
        impls.append(_ARC_IMPL_TC)
    return tuple(impls)


def _resolve_arc_impl(device: Any, impl: str | None) -> str:
    if impl is None:
        impl = os.environ.get(_ARC_IMPL_ENV, _ARC_IMPL_AUTO)
    normalized = impl.strip().lower()
    if normalized not in _ARC_IMPLS:
        raise ValueError(f"impl must be one of {sorted(_ARC_IMPLS)} or omitted; received {impl!r}")
    supported = set(arc_w4a16_supported_impls(device))
    if normalized != _ARC_IMPL_AUTO and normalized not in supported:
        raise ValueError(
            f"impl={normalized!r} is unsupported on device {device}; "
            f"supported implementations are {sorted(supported)}"
        )
    # "auto" stays on the HIP kernels: they stream the packed weights once, while the vendor path
    # first writes and re-reads an fp16 copy of the whole weight (4.5x the bytes), so it cannot win
    # at decode batch sizes.
    return normalized


def arc_w4a16_plan(
    *,
    batch: int,
    n: int,
    k: int,
    group_size: int,
    activation_dtype: Any = None,
    split_k_slices: int = 0,
    cu_count: int = 0,
    packet_format: int = 0,
    kernel: int = KERNEL_AUTO,
) -> dict[str, int]:
    """Launch plan: m_tile, workgroups, groups_per_workgroup, max_tile_contributors,
    workspace_bytes and slice_cols (columns of a tile per workgroup), for reference packets
    (packet_format 0) or the native formats (1 symmetric, 2 asymmetric), for a kernel choice
    (KERNEL_AUTO, KERNEL_DOT2, KERNEL_MFMA)."""
    native = native_module()
    return dict(
        native.arc_w4a16_plan(
            batch, n, k, group_size, _act_code(activation_dtype), split_k_slices, cu_count,
            packet_format, kernel,
        )
    )


def _act_code(dtype: Any) -> int:
    if dtype is None:
        return ACT_F16
    if isinstance(dtype, int):
        return dtype
    torch = _require_torch()
    if dtype == torch.float16:
        return ACT_F16
    if dtype == torch.bfloat16:
        return ACT_BF16
    raise TypeError(f"unsupported activation dtype {dtype}")


def arc_workspace(device: Any, nbytes: int) -> Any:
    """Zero-filled uint8 workspace of at least nbytes for (device, current stream), cached.

    The GEMV's split-K counters return to zero after every launch, so the buffer stays valid for
    later calls on the same stream. Calls on different streams get different buffers.
    """
    torch = _require_torch()
    key = (_device_index(device), _current_stream_ptr(device))
    ws = _ARC_WORKSPACE_CACHE.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(int(nbytes), 1 << 20)
        ws = torch.zeros(size, device=device, dtype=torch.uint8)
        _ARC_WORKSPACE_CACHE[key] = ws
    return ws


def _split_k_partials(*, device: Any, batch: int, n: int, split_k_slices: int) -> Any:
    torch = _require_torch()
    key = (_device_index(device), split_k_slices, batch, n)
    partials = _ARC_SPLIT_K_PARTIALS_CACHE.get(key)
    if partials is None:
        partials = torch.empty((split_k_slices, batch, n), device=device, dtype=torch.float32)
        _ARC_SPLIT_K_PARTIALS_CACHE[key] = partials
    return partials


def _weight_buffer(*, device: Any, n: int, k: int) -> Any:
    torch = _require_torch()
    key = (_device_index(device), n, k)
    weight = _ARC_WEIGHT_BUFFER_CACHE.get(key)
    if weight is None:
        weight = torch.empty((n, k), device=device, dtype=torch.float16)
        _ARC_WEIGHT_BUFFER_CACHE[key] = weight
    return weight


def _vendor_workspace(*, device: Any) -> Any:
    torch = _require_torch()
    key = (_device_index(device), _VENDOR_WORKSPACE_BYTES)
    ws = _ARC_VENDOR_WORKSPACE_CACHE.get(key)
    if ws is None:
        ws = torch.empty(_VENDOR_WORKSPACE_BYTES, device=device, dtype=torch.uint8)
        _ARC_VENDOR_WORKSPACE_CACHE[key] = ws
    return ws


def pack_arc_w4a16_packets(
    q_u8: torch.Tensor,
    alpha: torch.Tensor,
    beta: torch.Tensor,
    *,
    group_size: int,
    packets: torch.Tensor | None = None,
) -> torch.Tensor:
    """Reference: decode_quant_linear.py:685-732."""
    torch = _require_torch()
    native = _require_gpu_backend()
    _check_gpu_tensor(q_u8, name="q_u8", dtype=torch.uint8, ndim=2)
    _check_gpu_tensor(alpha, name="alpha", dtype=torch.float16, ndim=2)
    _check_gpu_tensor(beta, name="beta", dtype=torch.float16, ndim=2)

    n, packed_k = q_u8.shape
    k = packed_k * 2
    packet_stride = arc_packet_stride_bytes(group_size)
    if k % group_size != 0:
        raise ValueError("k must be divisible by group_size")
    num_groups = k // group_size
    if alpha.shape != (n, num_groups):
        raise ValueError("alpha must have shape [n, k // group_size]")
    if beta.shape != (n, num_groups):
        raise ValueError("beta must have shape [n, k // group_size]")
    if n % 128 != 0:
        raise ValueError("n must be divisible by 128")
    expected_shape = ((n // 128) * num_groups, packet_stride)

    if packets is None:
        packets = torch.empty(expected_shape, device=q_u8.device, dtype=torch.uint8)
    else:
        _check_gpu_tensor(packets, name="packets", dtype=torch.uint8, ndim=2)
        if tuple(packets.shape) != expected_shape:
            raise ValueError(f"packets must have shape {expected_shape}")

    _check_same_device(("q_u8", q_u8), ("alpha", alpha), ("beta", beta), ("packets", packets))
    native.pack_arc_w4a16_packets(
        q_u8.data_ptr(),
        alpha.data_ptr(),
        beta.data_ptr(),
        packets.data_ptr(),
        n,
        k,
        group_size,
        packet_stride,
        _current_stream_ptr(q_u8.device),
    )
    return packets


def compute_arc_w4a16_group_sums(
    activations: torch.Tensor,
    *,
    group_size: int,
    output: torch.Tensor | None = None,
) -> torch.Tensor:
    """Per-group fp32 activation sums [batch, k / group_size] (arc_w4a16.cu:124-158)."""
    torch = _require_torch()
    native = _require_gpu_backend()
    _check_gpu_tensor(activations, name="activations", dtype=torch.float16, ndim=2)
    batch, k = activations.shape
    if k % group_size != 0:
        raise ValueError("k must be divisible by group_size")
    shape = (batch, k // group_size)
    if output is None:
        output = torch.empty(shape, device=activations.device, dtype=torch.float32)
    else:
        _check_gpu_tensor(output, name="output", dtype=torch.float32, ndim=2)
        if tuple(output.shape) != shape:
            raise ValueError(f"output must have shape {shape}")
    native.compute_arc_w4a16_group_sums(
        activations.data_ptr(),
        output.data_ptr(),
        batch,
        k,
        group_size,
        _current_stream_ptr(activations.device),
    )
    return output


def arc_w4a16_forward(
    activations: torch.Tensor,
    packets: torch.Tensor,
    *,
    n: int,
    k: int,
    group_size: int,
    output: torch.Tensor | None = None,
    split_k_slices: int | None = None,
    partials: torch.Tensor | None = None,
    impl: str | None = None,
) -> torch.Tensor:
    """y[M, N] = x[M, K] . dequant(packets)^T. Reference: decode_quant_linear.py:735-898.

    split_k_slices: None picks the built-in plan, 1 forces one workgroup per tile over all of K,
    S > 1 runs the reference split-K protocol (fp32 partials [S, M, N], then a reduction), using
    ``partials`` when given.
    """
    torch = _require_torch()
    native = _require_gpu_backend()
    _check_gpu_tensor(
        activations, name="activations", dtype=(torch.float16, torch.bfloat16), ndim=2
    )
    _check_gpu_tensor(packets, name="packets", dtype=torch.uint8, ndim=2)

    batch = activations.shape[0]
    if activations.shape[1] != k:
        raise ValueError("activations.shape[1] must match k")
    packet_stride = arc_packet_stride_bytes(group_size)
    if k % group_size != 0:
        raise ValueError("k must be divisible by group_size")
    num_groups = k // group_size
    expected_packets = ((n // 128) * num_groups, packet_stride)
    if tuple(packets.shape) != expected_packets:
        raise ValueError(f"packets must have shape {expected_packets}")

    out_dtype = activations.dtype
    if output is None:
        output = torch.empty((batch, n), device=activations.device, dtype=out_dtype)
    else:
        _check_gpu_tensor(output, name="output", dtype=out_dtype, ndim=2)
        if tuple(output.shape) != (batch, n):
            raise ValueError(f"output must have shape {(batch, n)}")
    _check_same_device(("activations", activations), ("packets", packets), ("output", output))

    resolved = _resolve_arc_impl(activations.device, impl)
    if split_k_slices is not None and split_k_slices < 1:
        raise ValueError("split_k_slices must be positive")
    if resolved in (_ARC_IMPL_TC, _ARC_IMPL_MFMA) and split_k_slices not in {None, 1}:
        raise ValueError(f"split_k_slices is only supported by impl={_ARC_IMPL_SCALAR!r}")
    stream_ptr = _current_stream_ptr(activations.device)

    if resolved == _ARC_IMPL_TC:
        if out_dtype != torch.float16:
            raise TypeError("impl='tc' supports fp16 activations only")
        weight = _weight_buffer(device=activations.device, n=n, k=k)
        workspace = _vendor_workspace(device=activations.device)
        native.cublaslt_fp16_after_packet_dequant(
            activations.data_ptr(),
            packets.data_ptr(),
            output.data_ptr(),
            weight.data_ptr(),
            workspace.data_ptr(),
            workspace.numel(),
            batch,
            n,
            k,
            group_size,
            packet_stride,
            stream_ptr,
        )
        return output

    if split_k_slices is not None and split_k_slices > 1:
        if out_dtype != torch.float16:
            raise TypeError("the partials split-K protocol supports fp16 activations only")
        if partials is None:
            partials = _split_k_partials(
                device=activations.device, batch=batch, n=n, split_k_slices=split_k_slices
            )
        else:
            _check_gpu_tensor(partials, name="partials", dtype=torch.float32, ndim=3)
            if tuple(partials.shape) != (split_k_slices, batch, n):
                raise ValueError(f"partials must have shape {(split_k_slices, batch, n)}")
            _check_same_device(("activations", activations), ("partials", partials))
        native.arc_w4a16_forward_split_k(
            activations.data_ptr(),
            packets.data_ptr(),
            0,
            partials.data_ptr(),
            batch,
            n,
            k,
            group_size,
            packet_stride,
            split_k_slices,
            stream_ptr,
        )
        native.reduce_arc_w4a16_split_k_partials(
            partials.data_ptr(), output.data_ptr(), batch, n, split_k_slices, stream_ptr
        )
        return output

    act = _act_code(out_dtype)
    requested = 0 if split_k_slices is None else split_k_slices
    kernel = _IMPL_KERNEL[resolved]
    plan = native.arc_w4a16_plan(batch, n, k, group_size, act, requested, 0, 0, kernel)
    ws_bytes = int(plan["workspace_bytes"])
    ws_ptr = 0
    if ws_bytes > 0:
        ws = arc_workspace(activations.device, ws_bytes)
        ws_ptr = ws.data_ptr()
        ws_bytes = ws.numel()
    if kernel != KERNEL_AUTO:
        native.w4a16_forward_kernel(
            activations.data_ptr(), packets.data_ptr(), output.data_ptr(), ws_ptr, ws_bytes,
            batch, n, k, group_size, 0, act, requested, kernel, stream_ptr,
        )
        return output
    native.arc_w4a16_forward_ex(
        activations.data_ptr(),
        packets.data_ptr(),
        output.data_ptr(),
        ws_ptr,
        ws_bytes,
        batch,
        n,
        k,
        group_size,
        packet_stride,
        act,
        requested,
        stream_ptr,
    )
    return output


def dequant_w4a16_to_fp16(
    q_u8: torch.Tensor,
    alpha: torch.Tensor,
    beta: torch.Tensor,
    *,
    group_size: int,
    output: torch.Tensor | None = None,
) -> torch.Tensor:
    """W[n, k] = half_rn(alpha * q + beta). Reference: decode_quant_linear.py:901-941."""
    torch = _require_torch()
    native = _require_gpu_backend()
    _check_gpu_tensor(q_u8, name="q_u8", dtype=torch.uint8, ndim=2)
    _check_gpu_tensor(alpha, name="alpha", dtype=torch.float16, ndim=2)
    _check_gpu_tensor(beta, name="beta", dtype=torch.float16, ndim=2)
    n, packed_k = q_u8.shape
    k = packed_k * 2
    if k % group_size != 0:
        raise ValueError("k must be divisible by group_size")
    num_groups = k // group_size
    if alpha.shape != (n, num_groups):
        raise ValueError("alpha must have shape [n, k // group_size]")
    if beta.shape != (n, num_groups):
        raise ValueError("beta must have shape [n, k // group_size]")
    if output is None:
        output = torch.empty((n, k), device=q_u8.device, dtype=torch.float16)
    else:
        _check_gpu_tensor(output, name="output", dtype=torch.float16, ndim=2)
        if tuple(output.shape) != (n, k):
            raise ValueError(f"output must have shape {(n, k)}")
    _check_same_device(("q_u8", q_u8), ("alpha", alpha), ("beta", beta), ("output", output))
    native.dequant_w4a16_to_fp16(
        q_u8.data_ptr(),
        alpha.data_ptr(),
        beta.data_ptr(),
        output.data_ptr(),
        n,
        k,
        group_size,
        _current_stream_ptr(q_u8.device),
    )
    return output


def dequant_arc_w4a16_packets_to_fp16(
    packets: torch.Tensor,
    *,
    n: int,
    k: int,
    group_size: int,
    output: torch.Tensor | None = None,
) -> torch.Tensor:
    """W[n, k] fp16 from packets (arc_w4a16.cu:183-220, bound at python_module.cpp:188-197)."""
    torch = _require_torch()
    native = _require_gpu_backend()
    _check_gpu_tensor(packets, name="packets", dtype=torch.uint8, ndim=2)
    packet_stride = arc_packet_stride_bytes(group_size)
    if k % group_size != 0:
        raise ValueError("k must be divisible by group_size")
    expected = ((n // 128) * (k // group_size), packet_stride)
    if tuple(packets.shape) != expected:
        raise ValueError(f"packets must have shape {expected}")
    if output is None:
        output = torch.empty((n, k), device=packets.device, dtype=torch.float16)
    else:
        _check_gpu_tensor(output, name="output", dtype=torch.float16, ndim=2)
        if tuple(output.shape) != (n, k):
            raise ValueError(f"output must have shape {(n, k)}")
    native.dequant_arc_w4a16_packets_to_fp16(
        packets.data_ptr(),
        output.data_ptr(),
        n,
        k,
        group_size,
        packet_stride,
        _current_stream_ptr(packets.device),
    )
    return output


def cublaslt_fp16_after_dequant(
    activations: torch.Tensor,
    q_u8: torch.Tensor,
    alpha: torch.Tensor,
    beta: torch.Tensor,
    *,
    group_size: int,
    output: torch.Tensor | None = None,
    weight_buffer: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
) -> torch.Tensor:
    """Vendor baseline: dequant to fp16 then hipBLASLt. Reference: decode_quant_linear.py:944-1015
    (cuBLASLt); the reference name is kept for drop-in callers."""
    torch = _require_torch()
    native = _require_gpu_backend()
    _check_gpu_tensor(activations, name="activations", dtype=torch.float16, ndim=2)
    _check_gpu_tensor(q_u8, name="q_u8", dtype=torch.uint8, ndim=2)
    _check_gpu_tensor(alpha, name="alpha", dtype=torch.float16, ndim=2)
    _check_gpu_tensor(beta, name="beta", dtype=torch.float16, ndim=2)
    batch, k = activations.shape
    n, packed_k = q_u8.shape
    if packed_k * 2 != k:
        raise ValueError("q_u8.shape[1] must match activations.shape[1] / 2")
    if k % group_size != 0:
        raise ValueError("k must be divisible by group_size")
    num_groups = k // group_size
    if alpha.shape != (n, num_groups):
        raise ValueError("alpha must have shape [n, k // group_size]")
    if beta.shape != (n, num_groups):
        raise ValueError("beta must have shape [n, k // group_size]")
    if output is None:
        output = torch.empty((batch, n), device=activations.device, dtype=torch.float16)
    else:
        _check_gpu_tensor(output, name="output", dtype=torch.float16, ndim=2)
        if tuple(output.shape) != (batch, n):
            raise ValueError(f"output must have shape {(batch, n)}")
    if weight_buffer is None:
        weight_buffer = torch.empty((n, k), device=activations.device, dtype=torch.float16)
    else:
        _check_gpu_tensor(weight_buffer, name="weight_buffer", dtype=torch.float16, ndim=2)
        if tuple(weight_buffer.shape) != (n, k):
            raise ValueError(f"weight_buffer must have shape {(n, k)}")
    if workspace is None:
        workspace = torch.empty(8 * 1024 * 1024, device=activations.device, dtype=torch.uint8)
    else:
        _check_gpu_tensor(workspace, name="workspace", dtype=torch.uint8, ndim=1)
    _check_same_device(
        ("activations", activations),
        ("q_u8", q_u8),
        ("alpha", alpha),
        ("beta", beta),
        ("output", output),
        ("weight_buffer", weight_buffer),
        ("workspace", workspace),
    )
    native.cublaslt_fp16_after_dequant(
        activations.data_ptr(),
        q_u8.data_ptr(),
        alpha.data_ptr(),
        beta.data_ptr(),
        output.data_ptr(),
        weight_buffer.data_ptr(),
        workspace.data_ptr(),
        workspace.numel(),
        batch,
        n,
        k,
        group_size,
        _current_stream_ptr(activations.device),
    )
    return output


hipblaslt_fp16_after_dequant = cublaslt_fp16_after_dequant
