"""MI355X (gfx950) implementation of JointLoom's data-parallel hot path.

The product is the C-ABI library ``libjointloom.so`` (include/jointloom.h)
and the Python mirror of the reference's ``grid_world_cpp`` module in
``grid_world.py``.  ``synthetic`` generates the benchmark's seeded maps and
agent placements; ``ring`` is the HBM-resident expert-record ring.
"""
from .grid_world import (  # noqa: F401
    GridWorldSimulator,
    MapfGPTObservationBuilder,
    StatelessGridWorldSimulator,
    default_profile,
    parse_profile,
    profile,
)

__all__ = [
    "GridWorldSimulator",
    "MapfGPTObservationBuilder",
    "StatelessGridWorldSimulator",
    "default_profile",
    "parse_profile",
    "profile",
]
