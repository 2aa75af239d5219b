"""The C-ABI library loads and exports every symbol include/fk_w4a16.h declares; host-only
entry points (plan, argument validation) behave without a GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "fk_w4a16.h"
LIB = REPO / "fast-kernels_amd" / "fast_kernels" / "libfk_w4a16.so"


def _declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(fk_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib() -> ctypes.CDLL:
    if not LIB.exists():
        pytest.fail(f"{LIB} is missing: run python __graft_entry__.py")
    return ctypes.CDLL(str(LIB))


def test_header_declares_expected_entry_points() -> None:
    names = _declared()
    for ref in [
        "pack_arc_w4a16_packets",
        "compute_arc_w4a16_group_sums",
        "arc_w4a16_forward",
        "arc_w4a16_forward_split_k",
        "reduce_arc_w4a16_split_k_partials",
        "dequant_w4a16_to_fp16",
        "dequant_arc_w4a16_packets_to_fp16",
    ]:
        assert f"fk_{ref}" in names
    assert len(names) >= 14


def test_library_exports_every_declared_symbol(lib: ctypes.CDLL) -> None:
    for name in _declared():
        assert hasattr(lib, name), name


class Plan(ctypes.Structure):
    _fields_ = [
        ("m_tile", ctypes.c_int),
        ("workgroups", ctypes.c_int),
        ("groups_per_workgroup", ctypes.c_int),
        ("max_tile_contributors", ctypes.c_int),
        ("workspace_bytes", ctypes.c_size_t),
        ("slice_cols", ctypes.c_int),
        ("schedule", ctypes.c_int),
    ]


def _plan(lib, batch, n, k, g, act=0, split=0, cu=256):
    p = Plan()
    rc = lib.fk_arc_w4a16_plan_for(batch, n, k, g, act, split, cu, ctypes.byref(p))
    return rc, p


@pytest.mark.parametrize(
    "shape,want_runs_per_tile,want_slice_cols",
    [
        ((1, 10240, 4096, 128), 1, 64),   # 80 tiles -> 160 64-column slices
        ((1, 12288, 4096, 128), 1, 64),   # 96 tiles -> 192 64-column slices
        ((1, 22016, 4096, 128), 1, 128),  # 172 tiles: whole tiles over all of K, no fix-up
        ((1, 4096, 14336, 128), 2, 32),   # 112 groups: runs of 56, 4 slices -> 256 workgroups
        ((1, 1024, 16384, 128), 2, 32),   # 32 slices, runs of 64 groups -> 64 workgroups
    ],
)
def test_plan_policy_without_gpu(lib: ctypes.CDLL, shape, want_runs_per_tile, want_slice_cols) -> None:
    """One row over the reference packets where neither stream schedule applies (K/G below 64
    with slices that do not divide over the CUs, or per-tile runs that split K): per-tile runs."""
    batch, n, k, g = shape
    rc, p = _plan(lib, batch, n, k, g)
    assert rc == 0
    ng = k // g
    slices = (n // 128) * (128 // want_slice_cols)
    assert p.m_tile == 1
    assert p.slice_cols == want_slice_cols
    assert p.groups_per_workgroup == -(-ng // want_runs_per_tile)
    assert p.workgroups == -(-(slices * ng) // p.groups_per_workgroup)
    assert p.workgroups <= 256 or want_runs_per_tile == 1
    if want_runs_per_tile == 1:
        assert p.max_tile_contributors == 1 and p.workspace_bytes == 0
    else:
        assert p.workspace_bytes >= 65536 + (n // 128) * 128 * 4 * p.max_tile_contributors


def test_plan_batch_tiles_and_forced_split(lib: ctypes.CDLL) -> None:
    # 2-16 rows over the reference packets: the matrix-core stream kernel by packet quarters
    for batch in (2, 3, 7, 16):
        rc, p = _plan(lib, batch, 14336, 4096, 64)
        assert rc == 0 and (p.m_tile, p.schedule, p.slice_cols, p.workgroups) == (16, 2, 32, 224)
    # with a forced K split the per-tile kernels: matrix cores from 8 rows, dot2 m-tiles below
    rc, p = _plan(lib, 16, 14336, 4096, 64, split=1)
    assert rc == 0 and p.m_tile == 16 and p.schedule == 0
    rc, p = _plan(lib, 7, 14336, 4096, 64, split=1)
    assert rc == 0 and p.m_tile == 8
    rc, p = _plan(lib, 3, 14336, 4096, 64, act=1, split=1)
    assert rc == 0 and p.m_tile == 4
    # S = 7 slices of a 64-group tile: runs of ceil(64/7) = 10 groups straddle tile boundaries
    rc, p = _plan(lib, 1, 1024, 8192, 128, split=7)
    assert rc == 0 and p.groups_per_workgroup == 10 and p.slice_cols == 128
    assert p.workgroups == -(-(8 * 64) // 10)
    assert p.max_tile_contributors == 8


@pytest.mark.parametrize(
    "args",
    [
        (1, 100, 4096, 128),   # n not a multiple of 128
        (1, 128, 4000, 128),   # k not a multiple of G
        (1, 128, 4096, 96),    # unsupported group size
        (0, 128, 4096, 128),   # batch 0
    ],
)
def test_plan_rejects_bad_shapes(lib: ctypes.CDLL, args) -> None:
    rc, _ = _plan(lib, *args)
    assert rc == 1
    lib.fk_last_error.restype = ctypes.c_char_p
    assert lib.fk_last_error()


def test_validation_runs_before_any_device_call(lib: ctypes.CDLL) -> None:
    # Bad arguments are rejected (FK_ERR_INVALID_ARGUMENT) without touching the GPU, so this
    # works on a machine with no GPU at all.
    lib.fk_last_error.restype = ctypes.c_char_p
    fwd = lib.fk_arc_w4a16_forward
    rc = fwd(None, None, None, None, 1, 128, 256, 128, 999, None)
    assert rc == 1 and b"packet_stride_bytes" in lib.fk_last_error()
    rc = fwd(None, None, None, None, 1, 128, 256, 128, 128 * 64 + 512, None)
    assert rc == 1 and b"must not be null" in lib.fk_last_error()
    rc = lib.fk_arc_w4a16_forward_split_k(None, None, None, None, 1, 128, 256, 128, 8704, 1, None)
    assert rc == 1 and b"greater than 1" in lib.fk_last_error()
    rc = lib.fk_arc_w4a16_forward_split_k(None, None, None, None, 1, 128, 256, 128, 8704, 3, None)
    assert rc == 1 and b"exceed" in lib.fk_last_error()
    rc = lib.fk_reduce_arc_w4a16_split_k_partials(None, None, 1, 128, 1, None)
    assert rc == 1
    rc = lib.fk_arc_w4a16_forward_ex(None, None, None, None, 0, 1, 128, 256, 128, 8704, 5, 0, None)
    assert rc == 1 and b"activation_dtype" in lib.fk_last_error()


def test_pybind_module_mirrors_reference_names() -> None:
    from fast_kernels.native import native_build_info, native_module

    m = native_module()
    for name in [
        "build_info",
        "compute_arc_w4a16_group_sums",
        "pack_arc_w4a16_packets",
        "arc_w4a16_forward",
        "arc_w4a16_forward_split_k",
        "reduce_arc_w4a16_split_k_partials",
        "dequant_w4a16_to_fp16",
        "dequant_arc_w4a16_packets_to_fp16",
        "cublaslt_fp16_with_weight",
        "cublaslt_fp16_after_packet_dequant",
        "cublaslt_fp16_after_dequant",
        "arc_w4a16_forward_ex",
        "arc_w4a16_plan",
        "packet_stride_bytes",
        "pack_native_w4a16_packets",
        "convert_arc_to_native_packets",
        "convert_native_to_arc_packets",
        "arc_w4a16_forward_native",
    ]:
        assert hasattr(m, name), name
    info = native_build_info()
    assert info["available"] and info["compiled_with_hip"]
    with pytest.raises(ValueError):
        m.arc_w4a16_forward(
            activations_ptr=0, packets_ptr=0, group_sums_ptr=0, output_ptr=0, batch=1, n=128,
            k=256, group_size=64, packet_stride_bytes=1, stream_ptr=0,
        )


@pytest.mark.parametrize("group_size", [64, 128])
def test_packet_format_strides(lib: ctypes.CDLL, group_size: int) -> None:
    """Reference packets: codes (64*G) + alpha + beta (256 + 256) per 128 columns; native slabs:
    codes (16*G) + 16 records per 32 columns: 4 bytes of alphas, or 8 with the zero points."""
    from fast_kernels.ops import packet_stride_bytes

    want = {0: 64 * group_size + 512, 1: 16 * group_size + 64, 2: 16 * group_size + 128}
    for fmt, stride in want.items():
        assert lib.fk_packet_stride_bytes(group_size, fmt) == stride
        assert packet_stride_bytes(group_size, fmt) == stride
    assert packet_stride_bytes(group_size, "native_sym") == want[1]
    assert lib.fk_packet_stride_bytes(group_size, 3) == -1
    assert lib.fk_packet_stride_bytes(96, 1) == -1
    with pytest.raises(ValueError):
        packet_stride_bytes(group_size, "native")


def test_native_format_validation_without_gpu(lib: ctypes.CDLL) -> None:
    lib.fk_last_error.restype = ctypes.c_char_p
    rc = lib.fk_pack_native_w4a16_packets(None, None, None, None, 128, 256, 128, 0, None)
    assert rc == 1 and b"packet_format" in lib.fk_last_error()
    rc = lib.fk_pack_native_w4a16_packets(None, None, None, None, 128, 256, 128, 2, None)
    assert rc == 1 and b"must not be null" in lib.fk_last_error()
    rc = lib.fk_convert_arc_to_native_packets(None, None, 100, 256, 128, 1, None)
    assert rc == 1
    rc = lib.fk_convert_native_to_arc_packets(None, None, 128, 256, 128, 7, None)
    assert rc == 1 and b"packet_format" in lib.fk_last_error()
    rc = lib.fk_arc_w4a16_forward_native(None, None, None, None, 0, 1, 128, 256, 128, 5, 0, 0, None)
    assert rc == 1 and b"packet_format" in lib.fk_last_error()
    rc = lib.fk_arc_w4a16_forward_native(None, None, None, None, 0, 1, 128, 256, 128, 1, 0, 0, None)
    assert rc == 1 and b"must not be null" in lib.fk_last_error()


@pytest.mark.parametrize(
    "shape,want",
    [
        # (batch, n, k, G) -> (slice_cols, groups per workgroup, workgroups, schedule) on 256 CUs
        # schedule 0: per-slice runs, 1: slice pairs, 2: stream (whole slices per CU, one range)
        ((1, 8192, 8192, 128), (32, 64, 256, 2)),      # 256 slices: one per CU, streamed
        ((1, 10240, 8192, 128), (32, 80, 256, 2)),     # 70B qkv: 1 slice + a quarter slice per CU
        ((1, 10240, 4096, 128), (64, 32, 160, 1)),     # 320 slices in 160 pairs
        ((1, 12288, 4096, 128), (16, 96, 256, 2)),     # 7B qkv: 768 half-slices, 3 per CU
        ((1, 28672, 4096, 128), (32, 128, 224, 2)),    # 8B gate_up: 896 slices, 4 per CU on 224 CUs
        ((1, 12288, 8192, 128), (32, 96, 256, 2)),     # 1 slice + pieces of the 128 left over
        ((1, 22016, 4096, 128), (32, 32, 688, 0)),     # 7B gate_up: 344 pairs would fill 2 rounds unevenly
        ((2, 12288, 4096, 128), (32, 32, 384, 0)),     # pairs and stream for one row only
        ((4, 12288, 4096, 128), (32, 48, 256, 2)),     # four rows: matrix cores on the stream schedule
        ((1, 57344, 8192, 128), (32, 512, 224, 2)),    # 70B gate_up: 8 whole slices on 224 CUs
        ((1, 8192, 28672, 128), (32, 224, 256, 2)),    # 70B down: one slice of 224 groups per CU
        ((1, 8192, 28672 + 128, 128), (16, 450, 256, 2)),  # 225 groups: 2 half slices per CU,
                                                           # the last block of each partial
        ((1, 4096, 11008, 128), (16, 86, 256, 2)),     # 7B down, 86 groups: a half slice per CU
        ((1, 4096, 1920, 128), (32, 15, 128, 0)),      # 15 groups: less than one block, runs
        ((1, 4096, 4096, 128), (16, 32, 256, 2)),      # 128 slices: a half slice per CU
        ((1, 4096, 14336, 128), (16, 112, 256, 2)),    # 128 slices of 112 groups: halves, whole K
        ((2, 14336, 4096, 64), (32, 128, 224, 2)),     # config 3: 448 slices, 2 per CU on 224 CUs
        ((4, 14336, 4096, 64), (32, 128, 224, 2)),     # on the matrix cores, no pieces
        ((8, 14336, 4096, 64), (32, 128, 224, 2)),     # eight rows, the same stream plan
        ((16, 14336, 4096, 64), (32, 128, 224, 2)),    # sixteen rows, the same stream plan
        ((4, 12288, 4096, 64), (32, 96, 256, 2)),      # 384 slices: 1 slice + pieces, 4 rows
        ((16, 12288, 4096, 64), (128, 16, 384, 0)),    # the same at 16 rows: matrix-core tiles
    ],
)
def test_native_plan_policy_without_gpu(lib: ctypes.CDLL, shape, want) -> None:
    batch, n, k, g = shape
    p = Plan()
    assert lib.fk_w4a16_plan_for_format(batch, n, k, g, 0, 0, 256, 1, ctypes.byref(p)) == 0
    assert (p.slice_cols, p.groups_per_workgroup, p.workgroups, p.schedule) == want
    arc = Plan()
    assert lib.fk_w4a16_plan_for_format(batch, n, k, g, 0, 0, 256, 0, ctypes.byref(arc)) == 0
    rc, ref = _plan(lib, batch, n, k, g)
    assert rc == 0 and (arc.slice_cols, arc.workgroups) == (ref.slice_cols, ref.workgroups)
    # reference packets, from either planning entry point: per-tile runs, the whole-tile stream
    # schedule with a whole tile per CU, (one row, fewer tiles) the quarter schedule, or (2-16
    # rows) the matrix-core stream kernel by packet quarters where the native plan takes it
    assert arc.schedule == ref.schedule and arc.m_tile == ref.m_tile
    if batch != 1:
        assert arc.schedule == 0 or (arc.m_tile, arc.slice_cols, arc.workgroups) == (
            16, 32, p.workgroups)
    elif n // 128 >= 256:
        assert (arc.schedule, arc.slice_cols) == (2, 128)
    elif arc.schedule == 2:
        # quarters, or eighths when at most half as many quarters as CUs and K/G <= 32
        assert arc.slice_cols == (16 if g == 128 and n // 32 <= 128 and k // g <= 32 else 32)
    # a fix-up needs a workspace exactly when slices are shared (runs that do not cover whole
    # slices, or stream pieces)
    assert (p.workspace_bytes > 0) == (p.max_tile_contributors > 1)


def test_fused_entry_points_validate_without_gpu(lib: ctypes.CDLL) -> None:
    lib.fk_last_error.restype = ctypes.c_char_p
    f = ctypes.c_float
    rc = lib.fk_w4a16_forward_rmsnorm(None, None, f(1e-5), None, None, None, 0, 1, 128, 256, 128,
                                      0, 0, 0, None)
    assert rc == 1 and b"packet_format" in lib.fk_last_error()
    rc = lib.fk_w4a16_forward_rmsnorm(None, None, f(1e-5), None, None, None, 0, 1, 128, 256, 128,
                                      1, 0, 0, None)
    assert rc == 1 and b"must not be null" in lib.fk_last_error()
    rc = lib.fk_w4a16_forward_silu_mul(None, None, None, 1, 384, 256, 128, 1, 0, None, f(0.0), None)
    assert rc == 1 and b"256" in lib.fk_last_error()
    # one row: the stream kernel with the prologue fused (a slice per workgroup at 192 slices;
    # whole slices on a divisor grid), none at several rows or with a forced split
    p = Plan()
    assert lib.fk_w4a16_plan_rmsnorm(1, 6144, 4096, 128, 1, 0, 256, 1, ctypes.byref(p)) == 0
    assert (p.schedule, p.workgroups, p.groups_per_workgroup, p.workspace_bytes) == (2, 192, 32, 0)
    assert lib.fk_w4a16_plan_rmsnorm(1, 28672, 4096, 128, 1, 0, 256, 1, ctypes.byref(p)) == 0
    assert (p.schedule, p.workgroups, p.groups_per_workgroup) == (2, 224, 128)
    assert lib.fk_w4a16_plan_rmsnorm(1, 6144, 4096, 128, 1, 2, 256, 1, ctypes.byref(p)) == 0
    assert p.schedule != 2
    p = Plan()
    assert lib.fk_w4a16_plan_rmsnorm(16, 4096, 4096, 128, 0, 0, 256, 1, ctypes.byref(p)) == 0
    assert (p.m_tile, p.slice_cols) == (8, 32)
    assert lib.fk_w4a16_plan_rmsnorm(1, 4096, 4096, 128, 0, 0, 256, 0, ctypes.byref(p)) == 1


def test_kernel_choice_plans_without_gpu(lib: ctypes.CDLL) -> None:
    """FK_KERNEL_DOT2 keeps every batch on m-tiles of at most 8 rows, FK_KERNEL_MFMA puts every
    batch on 16-row tiles (on the stream schedule over 32-column slices where the slices divide
    over 7/8 of the CUs or more, or 3-8 rows with pieces; others over whole 128-column tiles), FK_KERNEL_AUTO is the forward's dispatch; another value is an
    invalid argument."""
    lib.fk_last_error.restype = ctypes.c_char_p
    for batch, n, kernel, want in [(16, 14336, 1, (8, 32)), (2, 14336, 2, (16, 32)),
                                   (2, 14336, 0, (16, 32)), (16, 14336, 0, (16, 32)),
                                   (4, 14336, 0, (16, 32)), (4, 14336, 2, (16, 32)),
                                   (2, 12288, 0, (2, 32)), (2, 12288, 2, (16, 128)),
                                   (16, 12288, 0, (16, 128))]:
        p = Plan()
        assert lib.fk_w4a16_plan_for_kernel(batch, n, 4096, 64, 0, 0, 256, 1, kernel,
                                            ctypes.byref(p)) == 0
        assert (p.m_tile, p.slice_cols) == want, (batch, kernel)
    p = Plan()
    assert lib.fk_w4a16_plan_for_kernel(2, 14336, 4096, 64, 0, 0, 256, 0, 3, ctypes.byref(p)) == 1
    assert b"kernel" in lib.fk_last_error()
    rc = lib.fk_w4a16_forward_kernel(None, None, None, None, 0, 1, 128, 256, 128, 0, 0, 0, 5, None)
    assert rc == 1 and b"kernel" in lib.fk_last_error()


@pytest.mark.parametrize("split", [1, 2, 4])
def test_forced_split_never_pairs_or_streams(lib: ctypes.CDLL, split: int) -> None:
    """A forced K split at shapes that would otherwise stream slice pairs (10240 x 4096) or take
    the stream schedule (8192 x 8192) plans per-slice runs of ceil(K/G/split) groups: the pair and
    stream kernels only take whole slices over all of K from the automatic policy."""
    for n, k in ((10240, 4096), (8192, 8192)):
        p = Plan()
        assert lib.fk_w4a16_plan_for_format(1, n, k, 128, 0, split, 256, 1, ctypes.byref(p)) == 0
        assert p.schedule == 0 and p.slice_cols == 32, (n, k, split)
        assert p.groups_per_workgroup == -(-(k // 128) // split)


NOALLOC_SCRATCH_BYTES = 8388608 + 65536  # FK_NOALLOC_SCRATCH_BYTES


def test_automatic_plans_fit_the_noalloc_scratch(lib: ctypes.CDLL) -> None:
    """fk_w4a16_forward_noalloc runs the automatic plan with a fixed per-device scratch array: every
    automatic plan of up to 16 activation rows and N up to 131072 must fit it, over every packet
    format, both group sizes and the CU counts of the gfx950 parts (and neighbours)."""
    assert f"#define FK_NOALLOC_SCRATCH_BYTES (8388608 + 65536)" in HEADER.read_text()
    lib.fk_w4a16_plan_for_format.argtypes = [ctypes.c_int] * 8 + [ctypes.POINTER(Plan)]
    worst = (0, None)
    ns = [128, 1024, 4096, 6144, 8192, 10240, 12288, 14336, 22016, 28672, 32768, 57344, 65536,
          131072]
    ks = [512, 1024, 4096, 8192, 11008, 14336, 28672, 32768]
    for batch in range(1, 17):
        for n in ns:
            for k in ks:
                for g in (64, 128):
                    if k % g:
                        continue
                    for fmt in (0, 1, 2):
                        for cu in (224, 256, 304):
                            p = Plan()
                            rc = lib.fk_w4a16_plan_for_format(batch, n, k, g, 0, 0, cu, fmt,
                                                              ctypes.byref(p))
                            assert rc == 0, (batch, n, k, g, fmt, cu)
                            if p.workspace_bytes > worst[0]:
                                worst = (p.workspace_bytes, (batch, n, k, g, fmt, cu))
    assert worst[0] <= NOALLOC_SCRATCH_BYTES, worst


@pytest.mark.parametrize(
    "n,k,g,grid,whole_groups,piece_groups",
    [
        (57344, 8192, 128, 224, 128, 0),  # 448 tiles: two whole tiles each on 224 CUs
        (49152, 8192, 128, 256, 64, 32),  # 384 tiles: one whole tile + 128 tiles x 16 blocks / 256
        (32768, 4096, 128, 256, 32, 0),   # 256 tiles: one whole tile each, no pieces
        (65536, 8192, 128, 256, 128, 0),  # two whole tiles each
        (40960, 2048, 64, 256, 32, 8),    # G = 64: blocks of 8 groups; 64 tiles x 4 blocks / 256
    ],
)
def test_reference_packet_stream_plan_without_gpu(lib: ctypes.CDLL, n, k, g, grid, whole_groups,
                                                  piece_groups) -> None:
    """One row over reference packets with at least one whole 128-column tile per CU takes the
    stream schedule (whole tiles over a divisor grid of at least 7/8 of the CUs, else whole tiles
    + pieces of the tiles left over); fewer tiles take the quarter schedule where it applies, else
    the runs."""
    rc, p = _plan(lib, 1, n, k, g)
    assert rc == 0
    assert (p.schedule, p.slice_cols, p.workgroups) == (2, 128, grid)
    assert p.groups_per_workgroup == whole_groups + piece_groups
    if piece_groups:
        assert p.workspace_bytes == 65536 + 256 * 2 * 128 * 4
    else:
        assert p.workspace_bytes == 0 and p.max_tile_contributors == 1
    rc, p = _plan(lib, 1, 10240, 4096, 128)  # 80 tiles, 32 groups: per-tile runs
    assert rc == 0 and p.schedule == 0


@pytest.mark.parametrize(
    "n,k,g,want",
    [
        # (unit columns, workgroups, groups per workgroup, fix-up workspace) on 256 CUs
        ((14336), 8192, 128, (32, 224, 2 * 64, False)),      # 448 slices: 2 each on 224 CUs
        ((12288), 8192, 128, (32, 256, 64 + 32, True)),       # 384 slices: 1 whole + pieces
        (10240, 8192, 128, (32, 256, 64 + 16, True)),          # 70B qkv: a slice and a block
        (8192, 8192, 128, (32, 256, 64, False)),               # 70B o
        (8192, 28672, 128, (32, 256, 224, False)),             # 70B down
        (4096, 8192, 128, (32, 128, 64, False)),               # one slice each, K not split
        (4096, 4096, 128, (16, 256, 32, False)),               # 7B o: one 16-column eighth each
        (2048, 4096, 128, (16, 128, 32, False)),               # 128 eighths
        (14336, 4096, 128, (32, 224, 64, False)),              # divisor grid (7/8 of the CUs)
        (10240, 8192, 64, (32, 256, 128 + 32, True)),          # G = 64: blocks of 32 groups
    ],
)
def test_reference_packet_quarter_plan_without_gpu(lib: ctypes.CDLL, n, k, g, want) -> None:
    """One row over reference packets with fewer whole 128-column tiles than CUs takes the
    quarter schedule (32-column quarters of the packets on the native stream split, or 16-column
    eighths for short K with at most half as many quarters as CUs); shapes with a whole tile per
    CU keep the whole-tile stream schedule."""
    rc, p = _plan(lib, 1, n, k, g)
    assert rc == 0
    assert (p.schedule, p.m_tile) == (2, 1)
    assert (p.slice_cols, p.workgroups, p.groups_per_workgroup, p.workspace_bytes > 0) == want
    if want[3]:
        assert p.workspace_bytes == 65536 + p.workgroups * 2 * 32 * 4
    rc, p = _plan(lib, 1, 57344, 8192, 128)
    assert rc == 0 and (p.schedule, p.slice_cols) == (2, 128)


def test_matrix_core_stream_k_parts_plans_are_consistent(lib: ctypes.CDLL) -> None:
    """Every matrix-core stream plan with K in parts (2-16 rows, rows too long to stage whole):
    the parts divide K/G into whole blocks (8 waves x 2 or 4 groups), every part has the same
    slice groups (workgroups = parts x groups, groups x whole slices = N / 32), the grid keeps to
    7/8 of the CUs or more, and the workspace holds the counters region and [parts, M, N] fp32
    partials within 6 MB; the same plan for both formats at one shape."""
    seen = 0
    for g in (64, 128):
        quantum = 8 * (4 if g == 64 else 2)
        for batch in (3, 4, 8, 13, 16):
            for n in (2048, 4096, 8192, 10240, 14336, 28672):
                for k in (8192, 11008 // 128 * 128, 14336, 28672):
                    if k % g:
                        continue
                    for cu in (224, 256, 304):
                        for fmt in (0, 2):
                            p = Plan()
                            assert lib.fk_w4a16_plan_for_format(batch, n, k, g, 0, 0, cu, fmt,
                                                                ctypes.byref(p)) == 0
                            if not (p.m_tile == 16 and p.schedule == 2 and
                                    p.max_tile_contributors > 1):
                                continue
                            seen += 1
                            parts, ng, slices = p.max_tile_contributors, k // g, n // 32
                            assert ng % parts == 0 and (ng // parts) % quantum == 0, (batch, n, k, g)
                            assert p.workgroups % parts == 0
                            groups = p.workgroups // parts
                            whole = p.groups_per_workgroup // (ng // parts)
                            assert groups * whole == slices, (batch, n, k, g, cu, p.workgroups)
                            assert 8 * p.workgroups >= 7 * cu and p.workgroups <= cu
                            assert p.workspace_bytes == 65536 + parts * batch * n * 4
                            assert parts * batch * n * 4 <= 6 << 20
    assert seen > 50
