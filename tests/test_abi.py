"""The C-ABI boundary (include/jointloom.h, libjointloom.so) without a GPU:
every declared entry point is exported, the ctypes mirror has the header's
struct layout (checked against gcc on the header itself), and the host-side
argument checks return the documented status codes before any device work.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "jointloom.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(jl_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from iclr_2027_jointoom_amd._abi import load_library

    return load_library()


def test_every_declared_entry_point_is_exported(lib):
    from iclr_2027_jointoom_amd._abi import SIGNATURES

    names = declared_functions()
    assert len(names) >= 18
    assert sorted(SIGNATURES) == names
    for name in names:
        assert getattr(lib, name) is not None


def test_streaming_probe_lives_in_the_bench_library_only(lib):
    """jl_hbm_stream (the benchmark's bandwidth probe) is exported by
    libjl_bench.so and not by the product library."""
    from iclr_2027_jointoom_amd.build import BENCH_OUTPUT

    assert not hasattr(lib, "jl_hbm_stream")
    probe = ctypes.CDLL(str(BENCH_OUTPUT))
    assert probe.jl_hbm_stream is not None
    assert "jl_hbm_stream" not in HEADER.read_text()


def test_version_and_error_strings(lib):
    assert lib.jl_version().decode().startswith("jointloom-gfx950")
    assert b"invalid argument" in lib.jl_error_string(-1)
    assert b"map profile" in lib.jl_error_string(-2)
    assert b"edge buffer" in lib.jl_error_string(-3)
    assert b"too many agents per env" in lib.jl_error_string(-4)
    assert lib.jl_error_string(0) == b"success"


def test_host_side_argument_checks_return_before_device_work(lib):
    from iclr_2027_jointoom_amd._abi import MagatDesc, MapfGPTDesc, SimDesc

    assert lib.jl_step(None, None) == -1
    assert lib.jl_encode_map(None, None, 1, 64, 64, None) == -1
    assert lib.jl_encode_map(1, 1, 1, 64, 48, None) == -2  # H must be a multiple of 32 up to 256
    sim = SimDesc(n_envs=1, n_agents=4, map_w=64, map_h=64, task_mode=1)
    assert lib.jl_step(ctypes.byref(sim), None) == -1  # null buffers
    for bad_h in (80, 288, 0):
        sim.map_h = bad_h
        assert lib.jl_step(ctypes.byref(sim), None) == -2, bad_h
    for good_h in (96, 160, 192, 224):  # every multiple of 32 is a profile (setup.py:34-38)
        sim.map_h = good_h
        assert lib.jl_step(ctypes.byref(sim), None) == -1, good_h  # passes the profile check
    b = MapfGPTDesc(n_envs=1, n_agents=4, map_w=300, map_h=64)
    assert lib.jl_mapfgpt_build_state(ctypes.byref(b), 1, 1, 1, 1, None) == -2
    assert lib.jl_mapfgpt_build_rows(ctypes.byref(b), None, None) == -1
    m = MagatDesc(n_envs=1, n_agents=4, map_w=64, map_h=64)
    assert lib.jl_magat_nodes(ctypes.byref(m), None) == -1
    assert lib.jl_energy_maps(None, None, None, 1, 1, 1, 64, 64, 0, None) == -1
    assert lib.jl_energy_maps(1, 1, None, 0, 1, 1, 64, 64, 0, None) == 0  # empty batch: nothing to do
    assert lib.jl_seed_rng(None, 4, 1, None) == -1
    assert lib.jl_decode_to_uint8(1, 1, 1, 17, None) == -1
    from iclr_2027_jointoom_amd._abi import RecordsDesc

    r = RecordsDesc(n_envs=2, n_agents=4, features=13, positions=16, actions=16, episode_start=16,
                    new_goals=16, goals=16, history=None, rows=16)
    assert lib.jl_expand_records(ctypes.byref(r), None) == -1  # 13 columns need the histories
    r.features, r.history = 9, 16
    assert lib.jl_expand_records(ctypes.byref(r), None) == -1
    r.features, r.positions = 8, 18  # positions are read as 32-bit words
    assert lib.jl_expand_records(ctypes.byref(r), None) == -1
    from iclr_2027_jointoom_amd._abi import StageUploadDesc

    u = StageUploadDesc(host_slot=16, staging=16, device_slot=16, slot_bytes=8)
    assert lib.jl_ring_upload_compact(ctypes.byref(u), None) == -1  # no staging event
    u.staging_free = 16
    u.records = RecordsDesc(n_envs=2, n_agents=4, features=13)
    assert lib.jl_ring_upload_compact(ctypes.byref(u), None) == -1  # slot smaller than its layout


def test_builder_rejects_misaligned_buffers(lib):
    """Buffers the build accesses 16 bytes at a time, and the build scratch
    (64-bit atomics on 128-byte lines), must be aligned: JL_ERR_ARG before
    any device work."""
    from iclr_2027_jointoom_amd._abi import MapfGPTDesc

    def desc(**kw):
        fields = dict(n_envs=1, n_agents=4, map_w=64, map_h=64, grid_bits=256, state_packed=256,
                      histories=256, labels=256, cost_to_go=256, goal_cache=256, tokens=256,
                      active_mask=256, diagnostics=256, agent_info=256, cost_tiles=256)
        fields.update(kw)
        return MapfGPTDesc(**fields)

    for name in ("state_packed", "cost_to_go", "cost_tiles", "tokens"):
        b = desc(**{name: 256 + 8})
        assert lib.jl_mapfgpt_build_state(ctypes.byref(b), 1, 1, 1, 1, None) == -1, name
        assert lib.jl_mapfgpt_build_rows(ctypes.byref(b), 1, None) == -1, name
        assert lib.jl_mapfgpt_build_rows_noalloc(ctypes.byref(b), 1, None) == -1, name
        assert lib.jl_mapfgpt_single_launch(ctypes.byref(b)) == 0, name
    b = desc(build_scratch=256 + 64)
    assert lib.jl_mapfgpt_build_state(ctypes.byref(b), 1, 1, 1, 1, None) == -1
    assert lib.jl_mapfgpt_single_launch(ctypes.byref(desc(build_scratch=256))) == 1


def test_ctypes_structs_match_the_c_layout(tmp_path):
    from iclr_2027_jointoom_amd._abi import (BUILD_SCRATCH_WORDS, GAVE_UP_WORD, MagatDesc, MapfGPTDesc,
                                             RecordsDesc, SimDesc, StageUploadDesc)

    structs = {"jl_sim_t": SimDesc, "jl_mapfgpt_t": MapfGPTDesc, "jl_magat_t": MagatDesc,
               "jl_records_t": RecordsDesc, "jl_stage_upload_t": StageUploadDesc}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for field, _ in py._fields_:
            lines.append(f'printf("{cname} {field} %zu\\n", offsetof({cname}, {field}));')
    lines.append('printf("macro JL_BUILD_SCRATCH_WORDS %d\\n", JL_BUILD_SCRATCH_WORDS);')
    lines.append('printf("macro JL_BUILD_SCRATCH_GAVE_UP_WORD %d\\n", JL_BUILD_SCRATCH_GAVE_UP_WORD);')
    lines += ["return 0; }"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    c = {(ln.split()[0], ln.split()[1]): int(ln.split()[2]) for ln in out if ln}
    assert c[("macro", "JL_BUILD_SCRATCH_WORDS")] == BUILD_SCRATCH_WORDS
    assert c[("macro", "JL_BUILD_SCRATCH_GAVE_UP_WORD")] == GAVE_UP_WORD
    for cname, py in structs.items():
        assert c[(cname, "size")] == ctypes.sizeof(py), cname
        for field, _ in py._fields_:
            assert c[(cname, field)] == getattr(py, field).offset, (cname, field)
