"""Drop-in module name of the reference extension (``import grid_world_cpp as ext``).

Exposes COMPILED_MAP_W/H and the three classes for the map profile named by
MAPF_CUDA_MAP_PROFILE (default 128x128), as bind.cpp:94-237 does, the
CostTracer functions of the online-RL tree's bind.cpp:96-98, plus
``profile(w, h)`` for other sizes in the same process.
"""
from iclr_2027_jointoom_amd.grid_world import default_profile as _default_profile
from iclr_2027_jointoom_amd.grid_world import profile  # noqa: F401

_P = _default_profile()
COMPILED_MAP_W = _P.COMPILED_MAP_W
COMPILED_MAP_H = _P.COMPILED_MAP_H
MapfGPTObservationBuilder = _P.MapfGPTObservationBuilder
GridWorldSimulator = _P.GridWorldSimulator
StatelessGridWorldSimulator = _P.StatelessGridWorldSimulator
costtracer_reward_goals = _P.costtracer_reward_goals
costtracer_observe = _P.costtracer_observe
costtracer_reset = _P.costtracer_reset
