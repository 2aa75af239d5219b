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
