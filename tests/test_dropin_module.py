"""The drop-in module name and its map profiles, without a GPU.

``import grid_world_cpp as ext`` (mapf_gpt_online.py:291, grids.py:10,
minimal_p0_mapf_gpt_resident_runner.py:65) gives COMPILED_MAP_W/H and the
classes for the profile MAPF_CUDA_MAP_PROFILE names, with the checks and
messages of the reference's setup.py:9-40: any width, a height that is a
multiple of 32, 128x128 when the variable is unset or empty.  This build's
kernels also cap both sides at 256.
"""
import importlib
import sys

import pytest

from iclr_2027_jointoom_amd.grid_world import SUPPORTED_H, parse_profile


@pytest.fixture
def fresh_import(monkeypatch):
    def load(profile_text):
        if profile_text is None:
            monkeypatch.delenv("MAPF_CUDA_MAP_PROFILE", raising=False)
        else:
            monkeypatch.setenv("MAPF_CUDA_MAP_PROFILE", profile_text)
        monkeypatch.delitem(sys.modules, "grid_world_cpp", raising=False)
        return importlib.import_module("grid_world_cpp")

    return load


def test_every_height_multiple_of_32_up_to_256_is_a_profile():
    assert SUPPORTED_H == (32, 64, 96, 128, 160, 192, 224, 256)
    for h in SUPPORTED_H:
        for w in (1, 17, 65, 96, 256):
            assert parse_profile(f"{w}x{h}") == (w, h)
    assert parse_profile(" 96X96 ") == (96, 96)


@pytest.mark.parametrize(
    "text,message",
    [
        ("96", "must look like '<width>x<height>'"),
        ("axb", "must contain integer width/height"),
        ("0x64", "must be positive"),
        ("64x-32", "must be positive"),
        ("64x48", "height must be a multiple of 32"),
        ("257x64", "1 <= W <= 256"),
        ("64x288", "1 <= W <= 256"),
    ],
)
def test_profile_errors_carry_the_reference_messages(text, message):
    with pytest.raises(ValueError, match=message):
        parse_profile(text)


@pytest.mark.parametrize("text,expected", [(None, (128, 128)), ("", (128, 128)), ("  ", (128, 128)),
                                           ("96x96", (96, 96)), ("65x160", (65, 160))])
def test_import_follows_the_environment(fresh_import, text, expected):
    ext = fresh_import(text)
    assert (ext.COMPILED_MAP_W, ext.COMPILED_MAP_H) == expected
    assert ext.COMPILED_MAP_H % 32 == 0
    for cls in (ext.GridWorldSimulator, ext.StatelessGridWorldSimulator, ext.MapfGPTObservationBuilder):
        assert (cls._MAP_W, cls._MAP_H) == expected
    # the module-level functions of the online-RL tree's bind.cpp:96-98
    for name in ("costtracer_reward_goals", "costtracer_observe", "costtracer_reset"):
        assert callable(getattr(ext, name))


def test_import_rejects_a_bad_profile(fresh_import):
    with pytest.raises(ValueError, match="multiple of 32"):
        fresh_import("64x50")


def test_bind_surface_of_each_class(fresh_import):
    """The methods and properties of bind.cpp:98-236 on the module's classes."""
    ext = fresh_import("96x96")
    builder = {"build_tokens", "build_tokens_from_state", "append_actions", "reset_histories", "tokens",
               "active_mask", "labels", "cost_to_go", "state_packed", "histories", "agent_at_cell",
               "diagnostics", "pyg_ptr", "goal_cache", "memory_tensors"}
    sim = {"init_rng", "run_initialization", "step_sim_only", "step_compact_only", "update_derived_state",
           "build_magat_plus_nodes", "finalize_magat_plus_graph", "build_magat_plus_inputs",
           "materialize_pyg_inputs", "step_and_build_pyg", "step", "update_actions", "set_real_map_extents",
           "load_state", "decode_to_uint8", "task_mode", "max_episode_steps", "pyg_builder_mode",
           "pyg_local_gather_impl", "resolved_pyg_builder_impl", "memory_tensors"}
    stateless = {"refresh_compact_state_from_raw_batch", "materialize_pyg_inputs", "update_derived_state",
                 "build_magat_plus_nodes", "finalize_magat_plus_graph", "build_magat_plus_inputs",
                 "setup_imitation_obs", "update_energy_maps", "pyg_builder_mode", "pyg_local_gather_impl",
                 "resolved_pyg_builder_impl", "memory_tensors"}
    for cls, names in ((ext.MapfGPTObservationBuilder, builder), (ext.GridWorldSimulator, sim),
                       (ext.StatelessGridWorldSimulator, stateless)):
        missing = sorted(n for n in names if not hasattr(cls, n))
        assert not missing, f"{cls.__name__} lacks {missing}"
    assert not hasattr(ext.MapfGPTObservationBuilder, "pyg_x")  # test_mapf_gpt_cuda.py:57-59
