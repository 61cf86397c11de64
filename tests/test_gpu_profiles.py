"""Map profiles whose height is a multiple of 32 but not of 64 or a power of
two (96, 160, 192, 224; setup.py:34-38 accepts every multiple of 32): the
step, the token build (single launch, two-launch with 64-row and 128-row
lanes, and the workgroup BFS beyond 128 rows), cost_to_go, and the MAGAT
energy fields, nodes and edges, against the C oracle.

Rows of 96, 160 and 224 columns end in half a 64-bit word of the BFS row
masks; the row loaders read only the row's own bitmap words.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

# (W, H, A): build path
SHAPES = [
    (40, 96, 64),    # 3,840 cells: single launch
    (96, 96, 100),   # two-launch, two rows per lane
    (100, 160, 80),  # two-launch, two rows per lane
    (21, 192, 40),   # 4,032 cells: single launch
    (18, 224, 30),   # 4,032 cells: single launch
    (130, 224, 120),  # workgroup BFS (four wavefronts of rows, the last two almost empty)
    (256, 160, 50),  # workgroup BFS (four wavefronts of rows)
]


@pytest.mark.parametrize("W,H,A", SHAPES)
def test_profile_step_tokens_and_magat_match_oracle(oracle, W, H, A):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions

    E, steps = 2, 4
    grids, starts, goals = make_batch(W * 7 + H, E, W, H, A)
    ext = profile(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * H, 3, "standard_mapf", 64)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    builder = ext.MapfGPTObservationBuilder(g, A)
    stateless = ext.StatelessGridWorldSimulator(g, A, 3)
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=64)
    osim.load_state(starts, goals)
    ob = oracle.OracleMapfGPT(grids, A)
    acts = random_actions(np.random.default_rng(W + H), steps, E, A)
    # the map bits themselves (grid_world_cuda.cu:112-183 layout)
    assert np.array_equal(sim.memory_tensors["grid_compressed"].cpu().numpy().view(np.uint32), osim.grid_bits)
    for s in range(steps):
        builder.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        ob.build_state(osim.cur_x.view(np.int16), osim.cur_y.view(np.int16), osim.goal_x.view(np.int16),
                       osim.goal_y.view(np.int16))
        a = torch.from_numpy(acts[s]).cuda()
        builder.append_actions(a)
        ob.append(acts[s])
        sim.update_actions(a)
        sim.step_sim_only()
        osim.step(acts[s])
        torch.cuda.synchronize()
        tag = f"{W}x{H} A{A} step {s}"
        assert np.array_equal(builder.tokens.cpu().numpy(), ob.tokens), tag
        assert np.array_equal(builder.histories.cpu().numpy().view(np.uint16), ob.histories), tag
        assert builder.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), tag
        assert np.array_equal(torch.stack((sim.cur_x, sim.cur_y), -1).cpu().numpy(), osim.positions()), tag
        assert np.array_equal(sim.state_packed.cpu().numpy().view(np.uint16), osim.state_packed), tag
        assert np.array_equal(sim.grid_ocp.cpu().numpy().view(np.uint32), osim.grid_ocp), tag
    assert np.array_equal(builder.cost_to_go.cpu().numpy().view(np.uint16), ob.cost_to_go)

    rows = osim.state_packed.view(np.int16).copy()
    rows_reset = rows.copy()
    rows_reset[:, 7] = 1
    stateless.update_energy_maps(torch.from_numpy(rows_reset).cuda(), len(rows_reset))
    stateless.refresh_compact_state_from_raw_batch(torch.from_numpy(rows).cuda())
    stateless.materialize_pyg_inputs()
    m = oracle.OracleMagat(grids, A)
    m.update_energy(rows_reset.view(np.uint16), len(rows_reset))
    m.refresh(rows.view(np.uint16))
    m.nodes()
    m.edges()
    torch.cuda.synchronize()
    assert np.array_equal(stateless.energy_maps.cpu().numpy(), m.energy)
    assert np.array_equal(stateless.pyg_x.cpu().numpy(), m.pyg_x)
    ei, ea = m.valid_edges()
    assert np.array_equal(stateless.pyg_edge_index.cpu().numpy(), ei)
    assert np.array_equal(stateless.pyg_edge_attr.cpu().numpy(), ea)


@pytest.mark.parametrize("H", [96, 160, 224])
def test_last_row_of_the_last_env_reads_no_word_past_its_bitmap(oracle, H):
    """Goals and agents in the last row of the last env, whose bitmap ends
    the tensor: that row's BFS mask ends in half a 64-bit word, and the
    loader reads only the row's own 32-bit words (the word after them would
    lie past the tensor).  Fields and tokens equal the oracle's."""
    from iclr_2027_jointoom_amd import profile

    E, W, A = 3, 48, 2
    grids = np.zeros((E, W, H), np.uint8)
    grids[:, W // 2, 1:] = 1  # a wall with a gap at y = 0
    ext = profile(W, H)
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)
    cur = np.array([[[0, 0], [W - 1, H - 1]]] * E, np.int16)
    gol = np.array([[[W - 1, H - 1], [W - 1, 0]]] * E, np.int16)
    t = [torch.from_numpy(np.ascontiguousarray(v)).cuda() for v in (cur[..., 0], cur[..., 1], gol[..., 0], gol[..., 1])]
    b.build_tokens_from_state(*t)
    ob = oracle.OracleMapfGPT(grids, A)
    ob.build_state(cur[..., 0], cur[..., 1], gol[..., 0], gol[..., 1])
    torch.cuda.synchronize()
    assert np.array_equal(b.cost_to_go.cpu().numpy().view(np.uint16), ob.cost_to_go)
    assert np.array_equal(b.tokens.cpu().numpy(), ob.tokens)
