"""ctypes binding of the C ABI declared in include/jointloom.h.

The descriptor structs mirror ``jl_sim_t``, ``jl_mapfgpt_t`` and
``jl_magat_t`` field for field.  ``load_library()`` loads the in-tree
``libjointloom.so`` built for gfx950 and raises when it is absent: there is no
CPU fallback on the product path.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

_PKG_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = _PKG_DIR / "libjointloom.so"
BUILD_SCRATCH_WORDS = 2080  # JL_BUILD_SCRATCH_WORDS of jointloom.h
GAVE_UP_WORD = 2  # JL_BUILD_SCRATCH_GAVE_UP_WORD of jointloom.h


def tiled_field_cells(map_w: int, map_h: int) -> int:
    """uint16 cells of one tiled distance field (cost_tiles of jl_mapfgpt_t):
    8x8 tiles over the map plus a one-tile border of unreachable cells."""
    return ((map_w + 7) // 8 + 2) * (map_h // 8 + 2) * 64

c_void_p = ctypes.c_void_p
c_int32 = ctypes.c_int32
c_int64 = ctypes.c_int64


class SimDesc(ctypes.Structure):
    """``jl_sim_t``: simulator state (GridWorldContext, grid_world_cuda.h:47-97)."""

    _fields_ = [
        ("n_envs", c_int32),
        ("n_agents", c_int32),
        ("map_w", c_int32),
        ("map_h", c_int32),
        ("task_mode", c_int32),
        ("max_episode_steps", c_int32),
        ("grid_bits", c_void_p),
        ("grid_ocp", c_void_p),
        ("cur_x", c_void_p),
        ("cur_y", c_void_p),
        ("goal_x", c_void_p),
        ("goal_y", c_void_p),
        ("actions", c_void_p),
        ("arrived", c_void_p),
        ("goal_changed", c_void_p),
        ("rewards", c_void_p),
        ("terminated", c_void_p),
        ("truncated", c_void_p),
        ("step_counts", c_void_p),
        ("state_packed", c_void_p),
        ("outcomes", c_void_p),
        ("free_cells", c_void_p),
        ("env_offsets", c_void_p),
        ("env_counts", c_void_p),
        ("rng_state", c_void_p),
        ("goal_candidates", c_void_p),
        ("candidate_cells", c_void_p),
        ("candidate_counts", c_void_p),
        ("goal_cursors", c_void_p),
        ("candidate_length", c_int32),
        ("candidate_stride", c_int32),
    ]


class MapfGPTDesc(ctypes.Structure):
    """``jl_mapfgpt_t``: MAPF-GPT builder buffers (mapf_gpt_builder.h:8-21)."""

    _fields_ = [
        ("n_envs", c_int32),
        ("n_agents", c_int32),
        ("map_w", c_int32),
        ("map_h", c_int32),
        ("grid_bits", c_void_p),
        ("state_packed", c_void_p),
        ("histories", c_void_p),
        ("labels", c_void_p),
        ("cost_to_go", c_void_p),
        ("agent_at_cell", c_void_p),
        ("goal_cache", c_void_p),
        ("tokens", c_void_p),
        ("active_mask", c_void_p),
        ("diagnostics", c_void_p),
        ("agent_info", c_void_p),
        ("cost_tiles", c_void_p),
        ("build_scratch", c_void_p),
        ("token_events", c_void_p * 2),
    ]


class MagatDesc(ctypes.Structure):
    """``jl_magat_t``: MAGAT builder buffers (grid_world_cuda.h:99-117)."""

    _fields_ = [
        ("n_envs", c_int32),
        ("n_agents", c_int32),
        ("map_w", c_int32),
        ("map_h", c_int32),
        ("grid_bits", c_void_p),
        ("grid_ocp", c_void_p),
        ("energy", c_void_p),
        ("states", c_void_p),
        ("pyg_x", c_void_p),
        ("pyg_pos", c_void_p),
        ("edge_counts", c_void_p),
        ("edge_prefix", c_void_p),
        ("num_edges", c_void_p),
        ("edge_index", c_void_p),
        ("edge_attr", c_void_p),
        ("edge_capacity", c_int64),
        ("env_edge_base", c_void_p),
    ]


class RecordsDesc(ctypes.Structure):
    """``jl_records_t``: one stage of compact expert records and the running
    goals/histories it expands against (frozen_stage_source.py:23-156)."""

    _fields_ = [
        ("n_envs", c_int32),
        ("n_agents", c_int32),
        ("features", c_int32),
        ("reserved", c_int32),
        ("positions", c_void_p),
        ("actions", c_void_p),
        ("episode_start", c_void_p),
        ("new_goals", c_void_p),
        ("goals", c_void_p),
        ("history", c_void_p),
        ("rows", c_void_p),
    ]


class StageUploadDesc(ctypes.Structure):
    """``jl_stage_upload_t``: one compact stage for the DMA thread's native step."""

    _fields_ = [
        ("host_slot", c_void_p),
        ("staging", c_void_p),
        ("device_slot", c_void_p),
        ("slot_bytes", c_int64),
        ("staging_free", c_void_p),
        ("rows_free", c_void_p),
        ("done", c_void_p),
        ("bytes_uploaded", c_int64),
        ("records", RecordsDesc),
    ]


# name -> (restype, argtypes); the exact set of symbols include/jointloom.h declares
SIGNATURES = {
    "jl_encode_map": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    "jl_step": (c_int32, [ctypes.POINTER(SimDesc), c_void_p]),
    "jl_update_actions": (c_int32, [ctypes.POINTER(SimDesc), c_void_p, c_void_p]),
    "jl_graph_retarget_actions": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, ctypes.POINTER(c_int32)]),
    "jl_goal_changed_scan": (c_int32, [ctypes.POINTER(SimDesc), c_void_p, c_void_p, c_void_p, c_void_p]),
    "jl_load_state": (
        c_int32,
        [ctypes.POINTER(SimDesc), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "jl_lifelong_init": (
        c_int32,
        [ctypes.POINTER(SimDesc), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "jl_seed_rng": (c_int32, [c_void_p, c_int64, ctypes.c_uint64, c_void_p]),
    "jl_mapfgpt_build_rows": (c_int32, [ctypes.POINTER(MapfGPTDesc), c_void_p, c_void_p]),
    "jl_mapfgpt_build_rows_noalloc": (c_int32, [ctypes.POINTER(MapfGPTDesc), c_void_p, c_void_p]),
    "jl_mapfgpt_build_state": (
        c_int32,
        [ctypes.POINTER(MapfGPTDesc), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "jl_mapfgpt_append_actions": (c_int32, [ctypes.POINTER(MapfGPTDesc), c_void_p, c_void_p]),
    "jl_mapfgpt_reset_histories": (c_int32, [ctypes.POINTER(MapfGPTDesc), c_void_p]),
    "jl_mapfgpt_cost_to_go": (c_int32, [ctypes.POINTER(MapfGPTDesc), c_void_p]),
    "jl_mapfgpt_agent_at_cell": (c_int32, [ctypes.POINTER(MapfGPTDesc), c_void_p]),
    "jl_energy_maps": (
        c_int32,
        [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,
         c_void_p],
    ),
    "jl_energy_maps_flagged": (
        c_int32, [ctypes.POINTER(SimDesc), c_void_p, c_int32, c_void_p, c_void_p, c_void_p]
    ),
    "jl_goal_changed_refresh": (
        c_int32, [ctypes.POINTER(SimDesc), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]
    ),
    "jl_magat_occupancy": (c_int32, [ctypes.POINTER(MagatDesc), c_void_p]),
    "jl_magat_nodes": (c_int32, [ctypes.POINTER(MagatDesc), c_void_p]),
    "jl_magat_edges": (c_int32, [ctypes.POINTER(MagatDesc), c_void_p]),
    "jl_mapfgpt_single_launch": (c_int32, [ctypes.POINTER(MapfGPTDesc)]),
    "jl_mapfgpt_refresh_state": (
        c_int32,
        [ctypes.POINTER(MapfGPTDesc), c_void_p, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "jl_costtracer_reward_goals": (
        c_int32,
        [ctypes.POINTER(SimDesc), ctypes.POINTER(MapfGPTDesc), c_void_p, c_void_p, c_int32, c_void_p,
         c_void_p, c_void_p, c_void_p],
    ),
    "jl_costtracer_observe": (
        c_int32, [ctypes.POINTER(SimDesc), ctypes.POINTER(MapfGPTDesc), c_void_p, c_void_p, c_void_p]
    ),
    "jl_costtracer_reset": (
        c_int32,
        [ctypes.POINTER(SimDesc), c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32,
         c_void_p],
    ),
    "jl_expand_records": (c_int32, [ctypes.POINTER(RecordsDesc), c_void_p]),
    "jl_ring_upload_compact": (c_int32, [ctypes.POINTER(StageUploadDesc), c_void_p]),
    "jl_decode_to_uint8": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p]),
    "jl_error_string": (ctypes.c_char_p, [c_int32]),
    "jl_version": (ctypes.c_char_p, []),
}

_LIB = None


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libjointloom.so (raises OSError/RuntimeError if it is missing)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    # torch's bundled libamdhip64.so.7 must be the process's HIP runtime, so
    # that the streams and device pointers torch hands out are valid here.
    import torch  # noqa: F401

    lib_path = Path(path) if path is not None else LIBRARY_PATH
    if not lib_path.exists():
        raise RuntimeError(
            f"{lib_path} is missing: build the gfx950 library first "
            "(python -c 'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(str(lib_path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if path is None:
        _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    """Raise RuntimeError for a non-zero status of an entry point."""
    if rc != 0:
        lib = load_library()
        msg = lib.jl_error_string(int(rc)).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {rc})")
