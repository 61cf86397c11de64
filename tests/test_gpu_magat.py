"""GPU parity of the MAGAT path (jl_energy_*, jl_magat_*) against the C oracle.

Ports /root/reference/tests/expert/test_compact_state_api.py and
test_cuda_kernels.py to the gfx950 path and adds oracle parity at the C4
shape (64x64, density 0.3, 256 agents) on fewer envs.  Bit-exact: energy
fields, occupancy, node features (float32, 0 ULP), positions, edge counts,
prefix, COO edges and attributes.
"""
import json
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def ext_for(w, h):
    from iclr_2027_jointoom_amd import profile

    return profile(w, h)


def _rows(E, A, starts, goals, reset):
    rows = np.zeros((E * A, 8), np.int16)
    blk = rows.reshape(E, A, 8)
    blk[:, :, 0] = np.arange(E)[:, None]
    blk[:, :, 1] = np.arange(A)[None, :]
    blk[:, :, 2:4] = starts
    blk[:, :, 4:6] = goals
    blk[:, :, 7] = reset
    return rows


def _compare(sim, m, tag=""):
    """Every MAGAT output of a simulator equals the oracle's."""
    torch.cuda.synchronize()
    pairs = [
        ("energy_maps", sim.energy_maps, m.energy),
        ("grid_ocp", sim.grid_ocp, m.grid_ocp.view(np.int32)),
        ("pyg_x", sim.pyg_x, m.pyg_x),
        ("pyg_pos", sim.pyg_pos, m.pyg_pos),
        ("edge_counts", sim.memory_tensors["edge_counts"], m.edge_counts),
        ("pyg_edge_prefix", sim.memory_tensors["pyg_edge_prefix"], m.edge_prefix),
        ("pyg_num_edges", sim.pyg_num_edges, m.num_edges),
    ]
    for name, got, exp in pairs:
        g = got.cpu().numpy()
        assert g.shape == exp.shape, f"{tag} {name} shape {g.shape} != {exp.shape}"
        assert np.array_equal(g, exp), f"{tag} {name} differs at {np.argwhere(g != exp)[:5].tolist()}"
    ei, ea = m.valid_edges()
    assert np.array_equal(sim.pyg_edge_index.cpu().numpy(), ei), f"{tag} edge_index"
    assert np.array_equal(sim.pyg_edge_attr.cpu().numpy(), ea), f"{tag} edge_attr"


def _oracle_stateless(oracle, grids, rows_reset, rows):
    E, W, H = grids.shape
    A = len(rows) // E
    m = oracle.OracleMagat(grids, A)
    m.update_energy(rows_reset.view(np.uint16), len(rows_reset))
    m.refresh(rows.view(np.uint16))
    m.nodes()
    m.edges()
    return m


@pytest.mark.parametrize(
    "E,W,A,density",
    [(4, 64, 256, 0.3), (3, 32, 64, 0.2), (2, 128, 300, 0.2), (1, 256, 160, 0.2), (1, 128, 1100, 0.1)],
)
def test_stateless_batches_match_oracle(oracle, E, W, A, density):
    """C4 shape on fewer envs (first case), plus the other map profiles."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(100 + W, E, W, W, A, density=density)
    ext = ext_for(W, W)
    sim = ext.StatelessGridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 3)
    rows_reset = _rows(E, A, starts, goals, 1)
    rows = _rows(E, A, starts, goals, 0)
    sim.update_energy_maps(torch.from_numpy(rows_reset).cuda(), len(rows_reset))
    sim.refresh_compact_state_from_raw_batch(torch.from_numpy(rows).cuda())
    sim.materialize_pyg_inputs()
    _compare(sim, _oracle_stateless(oracle, grids, rows_reset, rows), f"E{E} W{W} A{A}")


def test_edges_from_scanned_env_bases_match_oracle(oracle):
    """More than 8,192 edge slices (envs x 64-agent slices): the edge writer
    takes its env bases from the one-workgroup env scan instead of summing
    the node pass's slice totals itself.  8,200 envs of 4 agents on 32x32
    maps (eight generated batches repeated)."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 8200, 32, 4
    g8, s8, t8 = make_batch(321, 8, W, W, A, density=0.2)
    rep = (E + 7) // 8
    grids = np.tile(g8, (rep, 1, 1))[:E]
    starts = np.tile(s8, (rep, 1, 1))[:E]
    goals = np.tile(t8, (rep, 1, 1))[:E]
    ext = ext_for(W, W)
    sim = ext.StatelessGridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 3)
    rows_reset = _rows(E, A, starts, goals, 1)
    rows = _rows(E, A, starts, goals, 0)
    sim.update_energy_maps(torch.from_numpy(rows_reset).cuda(), len(rows_reset))
    sim.refresh_compact_state_from_raw_batch(torch.from_numpy(rows).cuda())
    sim.materialize_pyg_inputs()
    m = _oracle_stateless(oracle, grids, rows_reset, rows)
    assert int(m.num_edges[0]) > 0
    _compare(sim, m, f"E{E} W{W} A{A}")


def test_far_off_map_positions_match_oracle(oracle):
    """Positions far off the map: a cluster beyond +-8192 (the edge test then
    runs in 32-bit arithmetic) and two agents at the int16 extremes, whose
    squared distances to the others overflow int32 exactly as the
    reference's int arithmetic does (stateless_step.cu:517, :889)."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 2, 64, 40
    grids, starts, goals = make_batch(31, E, W, W, A, density=0.2)
    starts = starts.copy()
    starts[1, :10, 0] = 9000 + np.arange(10) % 4
    starts[1, :10, 1] = -9000 + np.arange(10) // 4
    starts[1, 10] = (-32768, 32767)
    starts[1, 11] = (-32766, 32765)
    ext = ext_for(W, W)
    sim = ext.StatelessGridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 3)
    rows_reset = _rows(E, A, starts, goals, 1)
    rows = _rows(E, A, starts, goals, 0)
    sim.update_energy_maps(torch.from_numpy(rows_reset).cuda(), len(rows_reset))
    sim.refresh_compact_state_from_raw_batch(torch.from_numpy(rows).cuda())
    sim.materialize_pyg_inputs()
    m = _oracle_stateless(oracle, grids, rows_reset, rows)
    assert m.edge_counts.reshape(E, A)[1, 10] > 0  # the overflow case is exercised
    _compare(sim, m, "far")


def test_partial_batch_and_invalid_rows_match_oracle(oracle):
    """Fewer rows than E*A (the rest filled with -1) and a refresh of only some agents."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 3, 64, 48
    grids, starts, goals = make_batch(5, E, W, W, A, density=0.3)
    ext = ext_for(W, W)
    sim = ext.StatelessGridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 3)
    m = oracle.OracleMagat(grids, A)
    rows_all = _rows(E, A, starts, goals, 1)
    sim.update_energy_maps(torch.from_numpy(rows_all).cuda(), len(rows_all))
    m.update_energy(rows_all.view(np.uint16), len(rows_all))
    # second round: new goals for every third agent, only those rows refreshed
    goals2 = goals.copy()
    goals2[:, ::3] = np.roll(goals[:, ::3], 1, axis=1)
    changed = _rows(E, A, starts, goals2, 1).reshape(E, A, 8)[:, ::3].reshape(-1, 8).copy()
    sim.update_energy_maps(torch.from_numpy(changed).cuda(), len(changed))
    m.update_energy(changed.view(np.uint16), len(changed))
    rows = _rows(E, A, starts, goals2, 0)[: 2 * A]  # env 2 absent: rows stay -1
    sim.refresh_compact_state_from_raw_batch(torch.from_numpy(rows).cuda())
    sim.materialize_pyg_inputs()
    m.refresh(rows.view(np.uint16))
    m.nodes()
    m.edges()
    _compare(sim, m, "partial")


def test_occupancy_kat():
    kat = json.loads((GOLDEN / "magat_kats.json").read_text())["occupancy"]
    ext = ext_for(128, 128)
    A = len(kat["agents"])
    sim = ext.StatelessGridWorldSimulator(torch.zeros((1, 128, 128), dtype=torch.int32, device="cuda"), A, 3)
    rows = _rows(1, A, np.asarray([kat["agents"]]), np.asarray([[kat["goal"]] * A]), 0)
    sim.refresh_compact_state_from_raw_batch(torch.from_numpy(rows).cuda())
    occ = sim.grid_ocp.cpu().numpy().view(np.uint32)[0]
    bit = lambda x, y: (int(occ[(x * 128 + y) >> 5]) >> ((x * 128 + y) & 31)) & 1  # noqa: E731
    assert all(bit(x, y) for x, y in kat["set"]) and not any(bit(x, y) for x, y in kat["unset"])
    assert torch.equal(sim.state_packed[:A].cpu(), torch.from_numpy(rows))


def test_local_gather_kats(oracle):
    """test_compact_state_api.py:262-358 on the 128x128 profile."""
    kat = json.loads((GOLDEN / "magat_kats.json").read_text())["local_gather"]
    A = kat["n_agents"]
    grid = np.zeros((1, 128, 128), np.int32)
    for x, y in kat["obstacles"]:
        grid[0, x, y] = 1
    ids = np.arange(A)
    pos = np.stack([ids // 16 + 40, ids % 16 + 40], 1)
    k = ids[256:] - 256
    pos[256:] = np.stack([k // 16 + 90, k % 16 + 90], 1)
    goals = np.full((A, 2), 64)
    for a, (px, py, gx, gy) in kat["overrides"].items():
        pos[int(a)] = (px, py)
        goals[int(a)] = (gx, gy)
    ext = ext_for(128, 128)
    sim = ext.StatelessGridWorldSimulator(torch.from_numpy(grid).cuda(), A, 3)
    rows_reset = _rows(1, A, pos[None], goals[None], 1)
    rows = _rows(1, A, pos[None], goals[None], 0)
    sim.update_energy_maps(torch.from_numpy(rows_reset).cuda(), A)
    sim.refresh_compact_state_from_raw_batch(torch.from_numpy(rows).cuda())
    sim.materialize_pyg_inputs()
    torch.cuda.synchronize()
    x = sim.pyg_x.view(A, 4, 13, 13).cpu()
    for agent, ch, r, c, v in kat["expected_x"]:
        assert x[agent, ch, r, c].item() == pytest.approx(v), (agent, ch, r, c)
    assert torch.equal(sim.pyg_pos.cpu(), torch.from_numpy(pos.astype(np.float32)))
    assert sim.pyg_num_edges.item() > 0
    _compare(sim, _oracle_stateless(oracle, grid.astype(np.uint8), rows_reset, rows), "kat")


# ---- test_cuda_kernels.py ports ---------------------------------------------------------------
def _kernel_states(num_agents, reset):
    data = torch.zeros((num_agents, 8), dtype=torch.int16, device="cuda")
    data[:, 1] = torch.arange(num_agents, dtype=torch.int16, device="cuda")
    data[:, 2] = 16 + torch.arange(num_agents, dtype=torch.int16, device="cuda")
    data[:, 3] = 16
    data[:, 4] = 48
    data[:, 5] = 48
    data[:, 7] = reset
    return data


def _stateless(num_envs, num_agents, w=128):
    ext = ext_for(w, w)
    return ext.StatelessGridWorldSimulator(torch.zeros((num_envs, w, w), dtype=torch.int32, device="cuda"),
                                           num_agents, 3)


@pytest.mark.parametrize("num_agents", [1, 4, 32])
def test_shapes_follow_runtime_agent_count(num_agents):
    sim = _stateless(1, num_agents)
    sim.update_energy_maps(_kernel_states(num_agents, 1), num_agents)
    sim.setup_imitation_obs(_kernel_states(num_agents, 0))
    torch.cuda.synchronize()
    assert sim.pyg_x.shape[0] == num_agents
    assert sim.pyg_pos.shape == (num_agents, 2)
    assert sim.pyg_ptr.tolist() == [0, num_agents]


def test_energy_map_marks_the_goal_cell():
    kat = json.loads((GOLDEN / "magat_kats.json").read_text())["energy_goal_cell"]
    sim = _stateless(1, 1)
    sim.update_energy_maps(_kernel_states(1, 1), 1)
    torch.cuda.synchronize()
    assert int(sim.energy_maps[0, 0, kat["goal"][0], kat["goal"][1]].item()) == kat["value"]


def test_edges_bounded_by_runtime_agent_count():
    sim = _stateless(1, 4)
    st = _kernel_states(4, 1)
    sim.update_energy_maps(st, 4)
    st[:, 7] = 0
    sim.setup_imitation_obs(st)
    torch.cuda.synchronize()
    edges = sim.pyg_edge_index
    assert edges.shape[0] == 2 and edges.numel() > 0
    assert int(edges.min()) >= 0 and int(edges.max()) < 4


def test_rejects_wrong_grid_shape_and_states():
    ext = ext_for(128, 128)
    with pytest.raises(RuntimeError):
        ext.StatelessGridWorldSimulator(torch.zeros((1, 129, 128), dtype=torch.int32, device="cuda"), 1, 3)
    sim = _stateless(1, 2)
    with pytest.raises(RuntimeError, match="int16"):
        sim.refresh_compact_state_from_raw_batch(torch.zeros((2, 8), dtype=torch.int32, device="cuda"))
    with pytest.raises(RuntimeError, match="8"):
        sim.refresh_compact_state_from_raw_batch(torch.zeros((2, 7), dtype=torch.int16, device="cuda"))
    with pytest.raises(RuntimeError, match="exceeds"):
        sim.refresh_compact_state_from_raw_batch(torch.zeros((3, 8), dtype=torch.int16, device="cuda"))


def test_stateless_memory_inventory_without_allocation():
    sim = _stateless(1, 4)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    inv = sim.memory_tensors
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == before
    assert {"grid_compressed", "energy_maps", "edge_counts", "pyg_edge_index_storage", "pyg_edge_attr_storage",
            "pyg_edge_prefix", "scan_temp_storage"} <= set(inv)
    assert (inv["pyg_edge_index"].untyped_storage().data_ptr()
            == inv["pyg_edge_index_storage"].untyped_storage().data_ptr())


def test_builder_mode_properties():
    """test_compact_state_api.py:39-63, 360-386 (non-128 profile: legacy rejected)."""
    sim = _stateless(1, 32)
    assert sim.pyg_builder_mode == "auto"
    assert sim.resolved_pyg_builder_impl in {"legacy_fullmap", "local_gather_scalar", "local_gather_async_sm89plus"}
    sim.pyg_builder_mode = "local_gather"
    for impl in ("scalar", "auto", "async_sm89plus"):
        sim.pyg_local_gather_impl = impl
        assert sim.pyg_local_gather_impl == impl
    small = _stateless(1, 64, w=64)
    with pytest.raises(RuntimeError, match="legacy_fullmap builder mode requires"):
        small.pyg_builder_mode = "legacy_fullmap"


def test_wrappers_match_each_other():
    """test_compact_state_api.py:87-112: every stateless entry point gives the same graph."""
    W, A = 128, 2
    a = _stateless(1, A)
    b = _stateless(1, A)
    st = torch.zeros((A, 8), dtype=torch.int16, device="cuda")
    st[:, 1] = torch.arange(A, dtype=torch.int16, device="cuda")
    st[:, 2] = torch.tensor([40, 41], dtype=torch.int16, device="cuda")
    st[:, 3] = torch.tensor([50, 51], dtype=torch.int16, device="cuda")
    st[:, 4] = torch.tensor([60, 61], dtype=torch.int16, device="cuda")
    st[:, 5] = torch.tensor([62, 63], dtype=torch.int16, device="cuda")
    st[:, 7] = 1
    a.update_energy_maps(st, A)
    b.update_derived_state(st, A)
    st[:, 7] = 0
    a.setup_imitation_obs(st)
    b.build_magat_plus_nodes(st)
    b.finalize_magat_plus_graph()
    torch.cuda.synchronize()
    assert torch.equal(b.state_packed[:A].cpu(), st.cpu())
    assert torch.equal(a.pyg_pos.cpu(), b.pyg_pos.cpu())
    assert torch.equal(a.pyg_x.cpu(), b.pyg_x.cpu())
    assert torch.equal(a.pyg_edge_index.cpu(), b.pyg_edge_index.cpu())
    assert torch.equal(a.pyg_edge_attr.cpu(), b.pyg_edge_attr.cpu())


# ---- stateful path ---------------------------------------------------------------------------
def test_stateful_standard_rollout_matches_oracle(oracle):
    """step_sim_only -> update_derived_state -> nodes -> graph, every step vs the oracle."""
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions

    E, W, A, steps = 3, 64, 256, 4
    grids, starts, goals = make_batch(77, E, W, W, A, density=0.3)
    ext = ext_for(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * W, 5, "standard_mapf", 64)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=64)
    osim.load_state(starts, goals)
    acts = random_actions(np.random.default_rng(1), steps, E, A)
    for s in range(steps):
        a = torch.from_numpy(acts[s]).cuda()
        sim.update_actions(a)
        if s % 2 == 0:
            sim.step()  # step_and_build_pyg
        else:
            sim.step_sim_only()
            sim.update_derived_state()
            sim.build_magat_plus_nodes()
            sim.finalize_magat_plus_graph()
        osim.step(acts[s])
        rows = osim.state_packed.copy()
        rows_reset = rows.copy()
        rows_reset[:, 7] = 1
        m = _oracle_stateless(oracle, grids, rows_reset.view(np.int16), rows.view(np.int16))
        _compare(sim, m, f"step {s}")
        assert np.array_equal(sim.state_packed.cpu().numpy(), rows.view(np.int16))
    # standard_mapf goals never change: no incremental refresh was needed
    assert int(sim.goal_changed_count.item()) == 0


def test_incremental_energy_refresh_matches_full_recompute():
    """test_compact_state_api.py:186-259 (lifelong mode)."""
    ext = ext_for(128, 128)
    A = 4
    grid = torch.zeros((1, 128, 128), dtype=torch.int32, device="cuda")
    sim = ext.GridWorldSimulator(grid, A, 2, 128 * 128, 1001)
    ref = ext.StatelessGridWorldSimulator(grid, A, 3)
    sim.run_initialization()
    sim.cur_x[0, :] = torch.tensor([10, 20, 30, 40], dtype=torch.int16, device="cuda")
    sim.cur_y[0, :] = torch.tensor([10, 20, 30, 40], dtype=torch.int16, device="cuda")
    sim.goal_x[0, :] = torch.tensor([11, 21, 31, 41], dtype=torch.int16, device="cuda")
    sim.goal_y[0, :] = torch.tensor([11, 21, 31, 41], dtype=torch.int16, device="cuda")
    sim.update_actions(torch.zeros((1, A), dtype=torch.uint8, device="cuda"))
    sim.step_compact_only()
    sim.update_derived_state()
    torch.cuda.synchronize()
    assert sim.goal_changed_count.item() == 0
    sim.cur_x[0, 0] = sim.goal_x[0, 0]
    sim.cur_y[0, 0] = sim.goal_y[0, 0]
    old_goal = (int(sim.goal_x[0, 0]), int(sim.goal_y[0, 0]))
    sim.step_compact_only()
    packed_after_step = sim.state_packed.clone()
    ref.update_energy_maps(packed_after_step, A)
    sim.update_derived_state()
    torch.cuda.synchronize()
    assert (int(sim.goal_x[0, 0]), int(sim.goal_y[0, 0])) != old_goal
    assert sim.goal_changed_flags.reshape(-1).sum().item() == 1
    assert sim.goal_changed_count.item() == 1
    assert torch.equal(sim.changed_state_packed[0].cpu(), sim.state_packed[0].cpu())
    assert torch.equal(sim.energy_maps.cpu(), ref.energy_maps.cpu())


@pytest.mark.parametrize("E,A,p", [(3, 37, 0.3), (2, 300, 0.05), (1, 5, 0.0), (512, 256, 0.02),
                                   (600, 256, 0.02), (1100, 256, 0.01), (520, 256, 0.0)])
def test_goal_changed_scan_and_packing(E, A, p):
    """update_derived_state after the first step: inclusive int64 cumsum of the
    flags, its total, changed rows packed at prefix - 1 with reset_flag 1 and
    the rest of the buffer cleared (grid_world_simulator.cpp:707-753,
    128_agents_map_step.cu:469-491); energy maps of the changed agents equal
    a stateless recompute, and with no flag set no field changes.  Up to
    131,072 agents this is one launch (scan, rows and fields together); the
    larger cases take the separate scan with two and four values per thread
    (more than 131,072 and 262,144 agents) and the flagged-field kernel."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(17 + A, E, 64, 64, A)
    ext = ext_for(64, 64)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 3, E * 64 * 64, 5, "standard_mapf", 64)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    sim.update_actions(torch.zeros((E, A), dtype=torch.uint8, device="cuda"))
    sim.step_sim_only()
    sim.update_derived_state()  # first step: full refresh
    sim.step_sim_only()
    sim.changed_state_packed.fill_(7)  # stale content the refresh must clear
    rng = np.random.default_rng(E * A)
    flags = (rng.random((E, A)) < p).astype(np.uint8)
    flags[flags != 0] += (rng.random(int(flags.sum())) < 0.2).astype(np.uint8)  # values, not booleans
    sim.goal_changed_flags.copy_(torch.from_numpy(flags).cuda())
    # move the flagged agents' goals so their fields change
    gx = sim.goal_x.cpu().numpy().copy()
    gy = sim.goal_y.cpu().numpy().copy()
    gx[flags != 0], gy[flags != 0] = starts[..., 0][flags != 0], starts[..., 1][flags != 0]
    sim.goal_x.copy_(torch.from_numpy(gx).cuda())
    sim.goal_y.copy_(torch.from_numpy(gy).cuda())
    before = sim.energy_maps.clone()
    sim.update_derived_state()
    torch.cuda.synchronize()
    prefix = np.cumsum(flags.reshape(-1).astype(np.int64))
    assert np.array_equal(sim.goal_changed_prefix.cpu().numpy(), prefix)
    assert int(sim.goal_changed_count.item()) == int(prefix[-1])
    expect = np.zeros((E * A, 8), np.int16)
    cx, cy = sim.cur_x.cpu().numpy(), sim.cur_y.cpu().numpy()
    acts = sim.actions.cpu().numpy()
    for gi in np.flatnonzero(flags.reshape(-1)):
        e, a = divmod(int(gi), A)
        expect[prefix[gi] - 1] = [e, a, cx[e, a], cy[e, a], gx[e, a], gy[e, a], acts[e, a], 1]
    assert np.array_equal(sim.changed_state_packed.cpu().numpy(), expect)
    # the flagged agents' fields are refreshed (a gap row left by a value above
    # 1 is not run: in the reference it would recompute env 0 agent 0)
    rows = expect[prefix[flags.reshape(-1) != 0] - 1]
    if len(rows):
        ref = ext.StatelessGridWorldSimulator(g, A, 3)
        ref.energy_maps.copy_(before)
        ref.update_energy_maps(torch.from_numpy(rows).cuda(), len(rows))
        torch.cuda.synchronize()
        assert torch.equal(sim.energy_maps.cpu(), ref.energy_maps.cpu())
    else:
        assert torch.equal(sim.energy_maps, before)


def test_more_than_256_agents():
    """test_compact_state_api.py:262-285."""
    A = 300
    sim = _stateless(1, A)
    ids = torch.arange(A, dtype=torch.int16, device="cuda")
    st = torch.zeros((A, 8), dtype=torch.int16, device="cuda")
    st[:, 1] = ids
    st[:, 2] = torch.div(ids, 20, rounding_mode="floor") + 10
    st[:, 3] = torch.remainder(ids, 20) + 10
    st[:, 4] = 64
    st[:, 5] = 64
    st[:, 7] = 1
    sim.update_energy_maps(st, A)
    st[:, 7] = 0
    sim.refresh_compact_state_from_raw_batch(st)
    sim.materialize_pyg_inputs()
    torch.cuda.synchronize()
    assert torch.equal(sim.pyg_pos.cpu(), st[:, 2:4].to(torch.float32).cpu())
    assert sim.pyg_num_edges.item() > 0


def test_c4_full_size_stateful(oracle):
    """BASELINE C4 shape (512 envs x 256 agents, 64x64, p = 0.3) through three
    stateful steps: node features, edge counts and edges of three sampled envs
    equal the oracle's, and over the whole batch the edge count is the sum of
    the counts, the prefix is their exclusive scan, edges are ordered by
    (source, target), stay within squared radius 49 inside one env, and their
    attributes are the position differences."""
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions

    E, W, A = 512, 64, 256
    grids, starts, goals = make_batch(78, E, W, W, A, density=0.3)
    ext = ext_for(W, W)
    sim = ext.GridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 0, E * W * W, 5,
                                 "standard_mapf", 256)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    sample = [0, 255, 511]
    acts = random_actions(np.random.default_rng(4), 3, E, A)
    for s in range(3):
        sim.update_actions(torch.from_numpy(acts[s]).cuda())
        sim.step_sim_only()
        sim.update_derived_state()
        sim.build_magat_plus_nodes()
        sim.finalize_magat_plus_graph()
        torch.cuda.synchronize()
        rows = sim.state_packed.cpu().numpy().reshape(E, A, 8)
        sub = rows[sample].copy()
        sub[:, :, 0] = np.arange(len(sample))[:, None]
        sub = sub.reshape(-1, 8)
        reset = sub.copy()
        reset[:, 7] = 1
        m = _oracle_stateless(oracle, grids[sample], reset, sub)
        k = len(sample)
        assert np.array_equal(sim.pyg_x.view(E, A, -1)[sample].cpu().numpy(), m.pyg_x.reshape(k, A, -1)), s
        counts = sim.memory_tensors["edge_counts"].view(E, A)
        assert np.array_equal(counts[sample].cpu().numpy(), m.edge_counts.reshape(k, A)), s
        ei = sim.pyg_edge_index
        ea = sim.pyg_edge_attr
        src_env = ei[0] // A
        m_ei, m_ea = m.valid_edges()
        for j, e in enumerate(sample):
            sel = src_env == e
            got = (ei[:, sel] - e * A + j * A).cpu().numpy()
            want_sel = (m_ei[0] // A) == j
            assert np.array_equal(got, m_ei[:, want_sel]), (s, e)
            assert np.array_equal(ea[sel].cpu().numpy(), m_ea[want_sel]), (s, e)
        # whole-batch properties
        flat = counts.reshape(-1).long()
        n = int(sim.pyg_num_edges.item())
        assert n == int(flat.sum().item()) == ei.shape[1]
        prefix = sim.memory_tensors["pyg_edge_prefix"]
        assert torch.equal(prefix[1:], flat.cumsum(0)) and int(prefix[0].item()) == 0
        key = ei[0] * (E * A) + ei[1]
        assert bool((key[1:] > key[:-1]).all())
        assert bool((ei[0] // A == ei[1] // A).all()) and bool((ei[0] != ei[1]).all())
        pos = sim.pyg_pos
        d = pos[ei[0]] - pos[ei[1]]
        assert torch.equal(ea[:, :2], d)
        assert torch.equal(ea[:, 2], d.abs().sum(1))
        assert bool(((d * d).sum(1) <= 49).all())
