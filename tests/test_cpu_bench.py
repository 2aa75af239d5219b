"""bench.py's split of the K timed steps into graph replays (CPU only)."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

from bench import rotations_for, step_chunk  # noqa: E402


@pytest.mark.parametrize(
    "steps,warmup,min_chunk,want",
    [
        (1000, 200, 3, (200, True)),   # defaults: five replays of the warm-up graph
        (20, 5, 3, (5, True)),         # four replays
        (20, 6, 3, (6, True)),         # three replays and a graph of the 2 left-over steps
        (20, 2, 3, (20, False)),       # warm-up too short to restart the weight copies
        (20, 0, 3, (20, False)),       # no warm-up: one graph
        (20, 20, 3, (20, False)),      # warm-up as long as the run: a graph of its own
        (20, 50, 3, (20, False)),
    ],
)
def test_step_chunk(steps: int, warmup: int, min_chunk: int, want) -> None:
    chunk, use = step_chunk(steps, warmup, min_chunk)
    assert (chunk, use) == want
    assert (steps // chunk) * chunk + steps % chunk == steps
    if use:
        assert chunk == warmup  # the warm-up is exactly one replay of the chunk graph


def test_min_chunk_spans_twice_the_infinity_cache() -> None:
    step_bytes = 441_460_000  # the 70B layer's four GEMVs
    m = rotations_for(step_bytes)
    assert m * step_bytes >= 2 * 256 * 2**20 and m == 3


@pytest.mark.parametrize(
    "chunk,r_min,min_chunk",
    [(5, 17, 3), (200, 17, 3), (200, 4, 3), (18, 17, 3), (35, 17, 3), (200, 64, 2), (1000, 9, 3),
     (7, 7, 3), (64, 21, 2)],
)
def test_step_rotations_keep_copies_cold_at_graph_restarts(chunk, r_min, min_chunk) -> None:
    from bench import step_rotations

    r = step_rotations(chunk, r_min, min_chunk)
    assert r >= r_min
    # Replay the copy sequence of three back-to-back replays of one graph: every copy must come
    # back no sooner than min_chunk steps (R steps inside a graph, chunk mod R at a restart).
    seq = [s % r for _ in range(3) for s in range(chunk)]
    last = {}
    for i, c in enumerate(seq):
        if c in last:
            assert i - last[c] >= min_chunk, (chunk, r, i, c)
        last[c] = i


def test_hbm_read_floor_probe_builds_for_gfx950(tmp_path) -> None:
    """The streaming-read probe behind the read floor (fast-kernels_amd/benchmarks/hbm_read_floor.hip,
    the source of the floor figures in the profiles) compiles for gfx950 with the library's flags,
    so the figures can be reproduced from the committed source."""
    import shutil
    import subprocess

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is not installed")
    src = Path(__file__).resolve().parents[1] / "fast-kernels_amd" / "benchmarks" / "hbm_read_floor.hip"
    out = tmp_path / "hbm_read_floor.o"
    proc = subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-Xclang", "-target-feature",
                           "-Xclang", "-packed-fp32-ops", "-c", str(src), "-o", str(out)],
                          capture_output=True, text=True, timeout=600)
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert out.stat().st_size > 0
