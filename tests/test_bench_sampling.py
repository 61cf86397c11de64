"""The bench's choice of the timed steps that carry the kernel's event pair:
one per block of EVENT_EVERY timed steps, inside the timed region, at the
block's middle step (never the region's first step unless it is the only one)."""

import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
import bench  # noqa: E402


@pytest.mark.parametrize("steps", [1, 2, 3, 9, 10, 11, 19, 20, 21, 50, 200, 201])
def test_one_sampled_step_per_block(steps):
    E = bench.EVENT_EVERY
    slots = bench.event_slots(steps)
    n = (steps + E - 1) // E
    assert sorted(slots.values()) == list(range(n))
    for step, block in slots.items():
        lo, hi = block * E, min((block + 1) * E, steps)
        assert lo <= step < hi
        assert step == lo + (hi - lo) // 2
    if steps > 1:
        assert 0 not in slots


def test_driver_command_samples_the_middle_of_each_half():
    # the driver's 20 timed steps: steps 5 and 15
    assert bench.event_slots(20) == {5: 0, 15: 1}
