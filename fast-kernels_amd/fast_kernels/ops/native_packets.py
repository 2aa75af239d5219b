"""Native gfx950 packet formats of the W4A16 decode linear, and the forward over them.

The reference packet (csrc/kernels/decode_quant_linear/arc_w4a16.cu:92-122) stores, per
128-column tile and group, the int4 code words of the 128 columns interleaved word row by word
row (512 bytes per row), then 128 fp16 alphas and 128 fp16 betas. Two things cost bandwidth on
MI355X: a workgroup that owns fewer than 128 columns (how the small decode shapes fill 256 CUs)
reads 128 bytes out of every 512, which HBM serves far below its streaming rate; and for int4
quantisation beta is always half_rn(-alpha * zp) with an integer zp in 0..15, so its 16 bits
carry at most 4.

The native formats store one slab per (tile, 32-column slice, group), in [tile][slice][group]
order, so the groups of a slice are one contiguous range:

  * code words: G/8 words per column (the reference's word packing, 8 codes along K per word),
    in the quarter order the kernels read (four lanes per column, 1 KB per wave-wide load);
  * 16 records, one per column pair (n, n + 16): the two fp16 alphas and, for "native_asym",
    the two negated zero points as fp16 (-zp[n], -zp[n + 16]), so one load brings a lane all the
    scales of its two columns and one packed fp16 multiply both betas.

"native_sym" (zp = 8) slabs are 16*G + 64 bytes, "native_asym" slabs 16*G + 128; a buffer is
[(N/32) * K/G, slab bytes]. The kernels rebuild beta = half_rn(-alpha * zp) bit for bit, so a
forward over native slabs returns exactly what the same launch over the reference packets they
came from returns. Slabs convert both ways on the GPU; converting reference packets whose betas
are not of that form raises ValueError instead of silently changing the weights.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Any

from fast_kernels.ops.decode_quant_linear import (
    _act_code,
    _check_gpu_tensor,
    _check_same_device,
    _current_stream_ptr,
    _require_gpu_backend,
    _require_torch,
    arc_packet_stride_bytes,
    arc_workspace,
)

if TYPE_CHECKING:  # pragma: no cover
    import torch

PACKET_ARC = 0
PACKET_NATIVE_SYM = 1
PACKET_NATIVE_ASYM = 2

PACKET_FORMATS: dict[str, int] = {
    "arc": PACKET_ARC,
    "native_sym": PACKET_NATIVE_SYM,
    "native_asym": PACKET_NATIVE_ASYM,
}


def packet_format_code(packet_format: str | int) -> int:
    if isinstance(packet_format, int) and packet_format in PACKET_FORMATS.values():
        return packet_format
    try:
        return PACKET_FORMATS[str(packet_format)]
    except KeyError as exc:
        raise ValueError(
            f"unsupported packet format {packet_format!r}; expected one of {sorted(PACKET_FORMATS)}"
        ) from exc


def packet_stride_bytes(group_size: int, packet_format: str | int) -> int:
    """Bytes per reference packet (code words 64*G, alphas 256, betas 256) or native slab (code
    words 16*G, then 16 records of 4 bytes (two alphas) or, for native_asym, 8 bytes (two alphas,
    two negated zero points as fp16))."""
    code = packet_format_code(packet_format)
    if code == PACKET_ARC:
        return arc_packet_stride_bytes(group_size)
    if group_size not in {64, 128}:
        raise ValueError("group_size must be 64 or 128")
    return 16 * group_size + (64 if code == PACKET_NATIVE_SYM else 128)


def _native_code(packet_format: str | int) -> int:
    code = packet_format_code(packet_format)
    if code == PACKET_ARC:
        raise ValueError("packet_format must be 'native_sym' or 'native_asym'")
    return code


def _packet_shape(n: int, k: int, group_size: int, code: int) -> tuple[int, int]:
    if k % group_size != 0:
        raise ValueError("k must be divisible by group_size")
    if n % 128 != 0:
        raise ValueError("n must be divisible by 128")
    rows_per_group = n // 128 if code == PACKET_ARC else n // 32
    return (rows_per_group * (k // group_size), packet_stride_bytes(group_size, code))


def _out_packets(packets: Any, shape: tuple[int, int], like: Any) -> Any:
    torch = _require_torch()
    if packets is None:
        return torch.empty(shape, device=like.device, dtype=torch.uint8)
    _check_gpu_tensor(packets, name="packets", dtype=torch.uint8, ndim=2)
    if tuple(packets.shape) != shape:
        raise ValueError(f"packets must have shape {shape}")
    return packets


def pack_native_w4a16_packets(
    q_u8: torch.Tensor,
    alpha: torch.Tensor,
    zero_points: torch.Tensor | None = None,
    *,
    group_size: int,
    packet_format: str | int = "native_sym",
    packets: torch.Tensor | None = None,
) -> torch.Tensor:
    """Native packets from q_u8 [N, K/2], alpha fp16 [N, K/G] and, for "native_asym",
    zero_points uint8 [N, K/G] with values 0..15 (weight = alpha * (q - zp))."""
    torch = _require_torch()
    native = _require_gpu_backend()
    code = _native_code(packet_format)
    _check_gpu_tensor(q_u8, name="q_u8", dtype=torch.uint8, ndim=2)
    _check_gpu_tensor(alpha, name="alpha", dtype=torch.float16, ndim=2)
    n, packed_k = q_u8.shape
    k = packed_k * 2
    shape = _packet_shape(n, k, group_size, code)
    if tuple(alpha.shape) != (n, k // group_size):
        raise ValueError("alpha must have shape [n, k // group_size]")
    zp_ptr = 0
    named = [("q_u8", q_u8), ("alpha", alpha)]
    if code == PACKET_NATIVE_ASYM:
        if zero_points is None:
            raise ValueError("packet_format 'native_asym' needs zero_points")
        _check_gpu_tensor(zero_points, name="zero_points", dtype=torch.uint8, ndim=2)
        if tuple(zero_points.shape) != (n, k // group_size):
            raise ValueError("zero_points must have shape [n, k // group_size]")
        zp_ptr = zero_points.data_ptr()
        named.append(("zero_points", zero_points))
    elif zero_points is not None:
        raise ValueError("packet_format 'native_sym' takes no zero_points (zp is 8)")
    packets = _out_packets(packets, shape, q_u8)
    named.append(("packets", packets))
    _check_same_device(*named)
    native.pack_native_w4a16_packets(
        q_u8.data_ptr(), alpha.data_ptr(), zp_ptr, packets.data_ptr(), n, k, group_size, code,
        _current_stream_ptr(q_u8.device),
    )
    return packets


def convert_arc_to_native_packets(
    arc_packets: torch.Tensor,
    *,
    n: int,
    k: int,
    group_size: int,
    packet_format: str | int = "native_sym",
    packets: torch.Tensor | None = None,
) -> torch.Tensor:
    """Reference packets -> native packets. Raises ValueError when some beta is not
    half_rn(-alpha * zp) for an integer zp in 0..15 (zp = 8 for "native_sym"). Synchronises the
    current stream (the check's flag is read back)."""
    torch = _require_torch()
    native = _require_gpu_backend()
    code = _native_code(packet_format)
    _check_gpu_tensor(arc_packets, name="arc_packets", dtype=torch.uint8, ndim=2)
    arc_shape = _packet_shape(n, k, group_size, PACKET_ARC)
    if tuple(arc_packets.shape) != arc_shape:
        raise ValueError(f"arc_packets must have shape {arc_shape}")
    packets = _out_packets(packets, _packet_shape(n, k, group_size, code), arc_packets)
    _check_same_device(("arc_packets", arc_packets), ("packets", packets))
    native.convert_arc_to_native_packets(
        arc_packets.data_ptr(), packets.data_ptr(), n, k, group_size, code,
        _current_stream_ptr(arc_packets.device),
    )
    return packets


def convert_native_to_arc_packets(
    native_packets: torch.Tensor,
    *,
    n: int,
    k: int,
    group_size: int,
    packet_format: str | int = "native_sym",
    packets: torch.Tensor | None = None,
) -> torch.Tensor:
    """Native packets -> reference packets (beta = half_rn(-alpha * zp)), bit for bit."""
    torch = _require_torch()
    native = _require_gpu_backend()
    code = _native_code(packet_format)
    _check_gpu_tensor(native_packets, name="native_packets", dtype=torch.uint8, ndim=2)
    shape = _packet_shape(n, k, group_size, code)
    if tuple(native_packets.shape) != shape:
        raise ValueError(f"native_packets must have shape {shape}")
    packets = _out_packets(packets, _packet_shape(n, k, group_size, PACKET_ARC), native_packets)
    _check_same_device(("native_packets", native_packets), ("packets", packets))
    native.convert_native_to_arc_packets(
        native_packets.data_ptr(), packets.data_ptr(), n, k, group_size, code,
        _current_stream_ptr(native_packets.device),
    )
    return packets


def arc_w4a16_forward_native(
    activations: torch.Tensor,
    packets: torch.Tensor,
    *,
    n: int,
    k: int,
    group_size: int,
    packet_format: str | int = "native_sym",
    output: torch.Tensor | None = None,
    split_k_slices: int | None = None,
) -> torch.Tensor:
    """y[M, N] = x[M, K] . dequant(packets)^T over packets of any format ("arc", "native_sym",
    "native_asym"); fp16 or bf16 activations, output in the same dtype. Same launch plan and
    results as ``arc_w4a16_forward`` with impl "scalar" over the equivalent reference packets."""
    torch = _require_torch()
    native = _require_gpu_backend()
    code = packet_format_code(packet_format)
    _check_gpu_tensor(
        activations, name="activations", dtype=(torch.float16, torch.bfloat16), ndim=2
    )
    _check_gpu_tensor(packets, name="packets", dtype=torch.uint8, ndim=2)
    batch = activations.shape[0]
    if activations.shape[1] != k:
        raise ValueError("activations.shape[1] must match k")
    shape = _packet_shape(n, k, group_size, code)
    if tuple(packets.shape) != shape:
        raise ValueError(f"packets must have shape {shape}")
    if output is None:
        output = torch.empty((batch, n), device=activations.device, dtype=activations.dtype)
    else:
        _check_gpu_tensor(output, name="output", dtype=activations.dtype, ndim=2)
        if tuple(output.shape) != (batch, n):
            raise ValueError(f"output must have shape {(batch, n)}")
    _check_same_device(("activations", activations), ("packets", packets), ("output", output))
    if split_k_slices is not None and split_k_slices < 1:
        raise ValueError("split_k_slices must be positive")
    requested = 0 if split_k_slices is None else int(split_k_slices)
    act = _act_code(activations.dtype)
    plan = native.arc_w4a16_plan(batch, n, k, group_size, act, requested, 0, code)
    ws_ptr, ws_bytes = 0, int(plan["workspace_bytes"])
    if ws_bytes > 0:
        ws = arc_workspace(activations.device, ws_bytes)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    native.arc_w4a16_forward_native(
        activations.data_ptr(), packets.data_ptr(), output.data_ptr(), ws_ptr, ws_bytes, batch,
        n, k, group_size, code, act, requested, _current_stream_ptr(activations.device),
    )
    return output


def arc_w4a16_forward_rmsnorm(
    activations: torch.Tensor,
    norm_weight: torch.Tensor,
    packets: torch.Tensor,
    *,
    n: int,
    k: int,
    group_size: int,
    eps: float = 1e-5,
    packet_format: str | int = "native_sym",
    output: torch.Tensor | None = None,
    split_k_slices: int | None = None,
) -> torch.Tensor:
    """y = rmsnorm(x) . W^T in one launch over native slabs, with
    rmsnorm(x) = round(norm_weight * round(x * rsqrt(mean(x^2) + eps))) in the activation dtype
    (the Llama input norm of the qkv and gate_up projections, rounded as an unfused norm kernel
    that writes its output would round it). norm_weight: [k], the activation dtype."""
    torch = _require_torch()
    native = _require_gpu_backend()
    code = _native_code(packet_format)
    _check_gpu_tensor(
        activations, name="activations", dtype=(torch.float16, torch.bfloat16), ndim=2
    )
    _check_gpu_tensor(norm_weight, name="norm_weight", dtype=activations.dtype, ndim=1)
    _check_gpu_tensor(packets, name="packets", dtype=torch.uint8, ndim=2)
    batch = activations.shape[0]
    if activations.shape[1] != k or norm_weight.shape[0] != k:
        raise ValueError("activations.shape[1] and norm_weight.shape[0] must match k")
    shape = _packet_shape(n, k, group_size, code)
    if tuple(packets.shape) != shape:
        raise ValueError(f"packets must have shape {shape}")
    if output is None:
        output = torch.empty((batch, n), device=activations.device, dtype=activations.dtype)
    else:
        _check_gpu_tensor(output, name="output", dtype=activations.dtype, ndim=2)
        if tuple(output.shape) != (batch, n):
            raise ValueError(f"output must have shape {(batch, n)}")
    _check_same_device(("activations", activations), ("norm_weight", norm_weight),
                       ("packets", packets), ("output", output))
    if split_k_slices is not None and split_k_slices < 1:
        raise ValueError("split_k_slices must be positive")
    requested = 0 if split_k_slices is None else int(split_k_slices)
    act = _act_code(activations.dtype)
    plan = native.w4a16_plan_rmsnorm(batch, n, k, group_size, act, requested, 0, code)
    ws_ptr, ws_bytes = 0, int(plan["workspace_bytes"])
    if ws_bytes > 0:
        ws = arc_workspace(activations.device, ws_bytes)
        ws_ptr, ws_bytes = ws.data_ptr(), ws.numel()
    native.w4a16_forward_rmsnorm(
        activations.data_ptr(), norm_weight.data_ptr(), float(eps), packets.data_ptr(),
        output.data_ptr(), ws_ptr, ws_bytes, batch, n, k, group_size, code, act, requested,
        _current_stream_ptr(activations.device),
    )
    return output


def arc_w4a16_forward_silu_mul(
    activations: torch.Tensor,
    packets: torch.Tensor,
    *,
    n: int,
    k: int,
    group_size: int,
    packet_format: str | int = "native_sym",
    output: torch.Tensor | None = None,
    norm_weight: torch.Tensor | None = None,
    eps: float = 1e-5,
) -> torch.Tensor:
    """silu(x . W_gate^T) * (x . W_up^T) in one launch, for native slabs of [W_gate; W_up]
    stacked along n (n rows in all, n % 256 == 0). Output [batch, n // 2] in the activation
    dtype; each GEMV result and the SiLU are rounded to it as the unfused pipeline rounds them.
    With norm_weight, x is first normalised as in arc_w4a16_forward_rmsnorm (a Llama block's input
    norm, gate_up projection and activation in one launch)."""
    torch = _require_torch()
    native = _require_gpu_backend()
    code = _native_code(packet_format)
    _check_gpu_tensor(
        activations, name="activations", dtype=(torch.float16, torch.bfloat16), ndim=2
    )
    _check_gpu_tensor(packets, name="packets", dtype=torch.uint8, ndim=2)
    batch = activations.shape[0]
    if activations.shape[1] != k:
        raise ValueError("activations.shape[1] must match k")
    if n % 256 != 0:
        raise ValueError("n (gate and up rows together) must be divisible by 256")
    shape = _packet_shape(n, k, group_size, code)
    if tuple(packets.shape) != shape:
        raise ValueError(f"packets must have shape {shape}")
    if output is None:
        output = torch.empty((batch, n // 2), device=activations.device, dtype=activations.dtype)
    else:
        _check_gpu_tensor(output, name="output", dtype=activations.dtype, ndim=2)
        if tuple(output.shape) != (batch, n // 2):
            raise ValueError(f"output must have shape {(batch, n // 2)}")
    _check_same_device(("activations", activations), ("packets", packets), ("output", output))
    norm_ptr = 0
    if norm_weight is not None:
        _check_gpu_tensor(norm_weight, name="norm_weight", dtype=activations.dtype, ndim=1)
        if norm_weight.shape[0] != k:
            raise ValueError("norm_weight.shape[0] must match k")
        _check_same_device(("activations", activations), ("norm_weight", norm_weight))
        norm_ptr = norm_weight.data_ptr()
    native.w4a16_forward_silu_mul(
        activations.data_ptr(), packets.data_ptr(), output.data_ptr(), batch, n, k, group_size,
        code, _act_code(activations.dtype), norm_ptr, float(eps),
        _current_stream_ptr(activations.device),
    )
    return output
