"""jl_mapfgpt_build_rows_noalloc, the MAPF-GPT build that allocates nothing
(its build scratch is the library's per-device static array), against
jl_mapfgpt_build_rows on identical builders: every output bit-exact, over
calls in a row through the C ABI whose env counts shrink and grow again (the
scratch keeps the previous call's contents), with rows whose diagnostics are
nonzero, and on a map whose build takes the two-launch path.  No call
allocates: torch's allocator and the device's free memory are unchanged
around each one (the first call of the process aside, which may set up the
HIP runtime's own state)."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

OUTPUTS = ("tokens", "labels", "active_mask", "cost_to_go", "state_packed", "histories", "goal_cache",
           "diagnostics")


def _rows(rng, grids, A, goals=None, bad=False):
    """Raw rows: every agent on a distinct random cell, goals on free cells
    unless given; with `bad`, a rejected row, two agents on one cell, a
    position off the map and a goal on an obstacle (nonzero diagnostics)."""
    E, W, H = grids.shape
    rows = np.zeros((E * A, 13), np.int64)
    rows[:, 0] = np.repeat(np.arange(E), A)
    rows[:, 1] = np.tile(np.arange(A), E)
    for e in range(E):
        cells = rng.choice(W * H, A, replace=False)
        rows[e * A:(e + 1) * A, 2] = cells // H
        rows[e * A:(e + 1) * A, 3] = cells % H
        if goals is None:
            free = np.flatnonzero(grids[e].ravel() == 0)
            g = rng.choice(free, A, replace=False)
            rows[e * A:(e + 1) * A, 4] = g // H
            rows[e * A:(e + 1) * A, 5] = g % H
    if goals is not None:
        rows[:, 4:6] = goals
    rows[:, 6] = rng.integers(0, 5, E * A)
    rows[:, 7] = 0 if goals is not None else 1
    rows[:, 8:13] = rng.integers(0, 6, (E * A, 5))
    if bad:
        rows[3, 0] = E + 1
        rows[7, 2:4] = rows[8, 2:4]
        rows[A + 1, 2] = W + 3
        rows[A + 5, 4:6] = np.argwhere(grids[1] != 0)[0]
    return torch.from_numpy(rows.astype(np.int16)).cuda()


def _noalloc_build(lib, builder, rows):
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.jl_mapfgpt_build_rows_noalloc(ctypes.byref(builder._desc), rows.data_ptr(), stream)
    assert rc == 0, rc


@pytest.mark.parametrize("W,H,sizes", [(64, 64, ((130, 64), (3, 40), (70, 64))), (128, 128, ((4, 24), (2, 16)))])
def test_noalloc_build_matches_build_rows(W, H, sizes):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd._abi import load_library

    lib = load_library()
    ext = profile(W, H)
    warmed = False  # the first call may set up HIP's own state (module, kernel arguments)
    for call, (E, A) in enumerate(sizes):
        print(f"noalloc build: map {W}x{H}, call {call}, E={E}, A={A}", flush=True)
        rng = np.random.default_rng(1000 * call + E + A)
        grids = (rng.random((E, W, H)) < 0.25).astype(np.int32)
        g = torch.from_numpy(grids).cuda()
        ref = ext.MapfGPTObservationBuilder(g, A)
        mine = ext.MapfGPTObservationBuilder(g, A)
        mine._desc.build_scratch = None  # the entry point must not need it
        assert ref.single_launch == (W * H <= 4096)
        first = _rows(rng, grids, A)
        goals = first.cpu().numpy()[:, 4:6].copy()
        for rows in (first, _rows(rng, grids, A, goals, bad=True)):
            ref.build_tokens(rows)
            torch.cuda.synchronize()
            before = torch.cuda.memory_allocated()
            free_before = torch.cuda.mem_get_info()[0]
            _noalloc_build(lib, mine, rows)
            torch.cuda.synchronize()
            # nothing from torch's allocator, and (after the first call) no
            # device memory from anywhere else in the process either
            assert torch.cuda.memory_allocated() == before
            if warmed:
                assert torch.cuda.mem_get_info()[0] == free_before, (call, "device memory was allocated")
            warmed = True
            for name in OUTPUTS:
                assert torch.equal(getattr(ref, name), getattr(mine, name)), (call, name)
        assert mine.diagnostics.abs().sum().item() > 0, call
        assert len(np.unique(mine.tokens.cpu().numpy()[:, 130])) > 2, call  # greedy tokens vary


def test_noalloc_build_rejects_what_build_rows_rejects():
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd._abi import load_library

    lib = load_library()
    ext = profile(64, 64)
    g = torch.zeros((2, 64, 64), dtype=torch.int32, device="cuda")
    b = ext.MapfGPTObservationBuilder(g, 8)
    rows = torch.zeros((16, 13), dtype=torch.int16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.jl_mapfgpt_build_rows_noalloc(None, rows.data_ptr(), stream) == -1
    assert lib.jl_mapfgpt_build_rows_noalloc(ctypes.byref(b._desc), None, stream) == -1
    b._desc.map_h = 48
    assert lib.jl_mapfgpt_build_rows_noalloc(ctypes.byref(b._desc), rows.data_ptr(), stream) == -2
    b._desc.map_h = 64
    b._desc.tokens = b._desc.tokens + 4  # misaligned wide buffer
    assert lib.jl_mapfgpt_build_rows_noalloc(ctypes.byref(b._desc), rows.data_ptr(), stream) == -1
