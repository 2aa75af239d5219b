"""The HIP library against the committed golden vectors (tests/golden/w4a16_golden.npz).

kat_* cases are exact: every product and partial sum is an integer multiple of the power-of-two
scale and below 2^24 of it, so fp32 accumulation in any order is exact and the GPU output must
equal the known answer bit-for-bit, for fp16 and for bf16 activations (x in {-2..2} is exact in
both; the bf16 answer is the exact value rounded once to bf16). rnd_* cases must match the frozen
oracle outputs: dequant and packets bit-exact, y within rtol 1e-2 / atol 1e-2*sqrt(K)*max|alpha|.
"""

from __future__ import annotations

import hashlib
import math

import numpy as np
import pytest

from conftest import gpu_available
from golden_vectors import load_cases, meta

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not gpu_available(), reason="needs a GPU"),
]

torch = pytest.importorskip("torch")

from fast_kernels.benchmarking.inputs import (  # noqa: E402
    bf16_bits_to_f32,
    f16_bits_to_f32,
    f32_to_bf16_bits,
)
from fast_kernels.native import native_module  # noqa: E402
from fast_kernels.ops import (  # noqa: E402
    arc_packet_stride_bytes,
    arc_w4a16_forward,
    arc_workspace,
    dequant_w4a16_to_fp16,
    pack_arc_w4a16_packets,
)

CASES = load_cases()
KAT = sorted(k for k in CASES if k.startswith("kat_"))
RND = sorted(k for k in CASES if k.startswith("rnd_"))


def _t16(bits: np.ndarray, dtype) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(dtype)


def _bits(t) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _weights(c):
    q = torch.from_numpy(c["q_u8"]).cuda()
    return q, _t16(c["alpha"], torch.float16), _t16(c["beta"], torch.float16)


@pytest.mark.parametrize("split", [0, -1])
@pytest.mark.parametrize("act", ["f16", "bf16"])
@pytest.mark.parametrize("name", KAT)
def test_known_answers_bit_exact(name: str, act: str, split: int) -> None:
    c = CASES[name]
    batch, n, k, g, _, _ = meta(c)
    q, a, b = _weights(c)
    w = dequant_w4a16_to_fp16(q, a, b, group_size=g)
    np.testing.assert_array_equal(_bits(w), c["dequant"])
    packets = pack_arc_w4a16_packets(q, a, b, group_size=g)
    x32 = f16_bits_to_f32(c["x"])
    y_exact = f16_bits_to_f32(c["y"]).astype(np.float32)
    if act == "f16":
        x, want = _t16(c["x"], torch.float16), c["y"]
    else:
        x, want = _t16(f32_to_bf16_bits(x32), torch.bfloat16), f32_to_bf16_bits(y_exact)
    split = (k // g) if split < 0 else split
    if split == 0:
        y = arc_w4a16_forward(x, packets, n=n, k=k, group_size=g)
    else:
        # One group per workgroup: every tile is finished from the partials of NG workgroups.
        native = native_module()
        act_code = 0 if act == "f16" else 1
        plan = native.arc_w4a16_plan(batch, n, k, g, act_code, split, 0)
        assert plan["max_tile_contributors"] > 1
        ws = arc_workspace(x.device, plan["workspace_bytes"])
        y = torch.empty((batch, n), device=x.device, dtype=x.dtype)
        native.arc_w4a16_forward_ex(
            x.data_ptr(), packets.data_ptr(), y.data_ptr(), ws.data_ptr(), ws.numel(), batch, n,
            k, g, arc_packet_stride_bytes(g), act_code, split, torch.cuda.current_stream().cuda_stream,
        )
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_bits(y), want)


@pytest.mark.parametrize("name", RND)
def test_frozen_oracle_outputs(name: str) -> None:
    c = CASES[name]
    batch, n, k, g, act, _ = meta(c)
    q, a, b = _weights(c)
    w = _bits(dequant_w4a16_to_fp16(q, a, b, group_size=g))
    assert hashlib.sha256(w.tobytes()).digest() == c["dequant_sha256"].tobytes()
    packets = pack_arc_w4a16_packets(q, a, b, group_size=g)
    torch.cuda.synchronize()
    assert hashlib.sha256(packets.cpu().numpy().tobytes()).digest() == c["packets_sha256"].tobytes()
    dtype = torch.float16 if act == "f16" else torch.bfloat16
    y = arc_w4a16_forward(_t16(c["x"], dtype), packets, n=n, k=k, group_size=g)
    torch.cuda.synchronize()
    conv = f16_bits_to_f32 if act == "f16" else bf16_bits_to_f32
    got = conv(_bits(y)).astype(np.float64)
    ref = conv(c["y"]).astype(np.float64)
    atol = 1e-2 * math.sqrt(k) * float(f16_bits_to_f32(c["alpha"]).max())
    assert np.all(np.abs(got - ref) <= atol + 1e-2 * np.abs(ref))
