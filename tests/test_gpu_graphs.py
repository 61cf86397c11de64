"""HIP-graph replay of the resident loops equals the eager loop, replay by
replay, with eager work and host synchronisation between the replays."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _setup(E, W, A, seed, density=0.2):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(seed, E, W, W, A, density=density)
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 3, E * W * W, 3, "standard_mapf", 1 << 20)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    return ext, g, sim, starts


def test_mapf_gpt_resident_graph_matches_eager():
    from iclr_2027_jointoom_amd.graphs import MapfGPTResidentGraph

    E, W, A = 8, 64, 64
    ext, g, sim_e, starts = _setup(E, W, A, 31)
    _, _, sim_g, _ = _setup(E, W, A, 31)
    b_e = ext.MapfGPTObservationBuilder(g, A)
    b_g = ext.MapfGPTObservationBuilder(g, A)
    rng = np.random.default_rng(4)

    def eager(sim, b, acts):
        b.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        b.append_actions(acts)
        sim.update_actions(acts)
        sim.step_sim_only()

    first = torch.from_numpy(rng.integers(0, 5, (E, A), dtype=np.uint8)).cuda()
    eager(sim_e, b_e, first)
    eager(sim_g, b_g, first)
    graph = MapfGPTResidentGraph(sim_g, b_g)
    for it in range(6):
        if it == 3:
            # a changed goal: the captured build refreshes that field on the device
            for sim in (sim_e, sim_g):
                sim.goal_x[1, 5] = int(starts[1, 7, 0])
                sim.goal_y[1, 5] = int(starts[1, 7, 1])
        acts = torch.from_numpy(rng.integers(0, 5, (E, A), dtype=np.uint8)).cuda()
        eager(sim_e, b_e, acts)
        graph.actions.copy_(acts)
        graph.replay()
        torch.cuda.synchronize()
        for name in ("tokens", "histories", "active_mask", "state_packed", "diagnostics", "goal_cache"):
            assert torch.equal(getattr(b_e, name), getattr(b_g, name)), (it, name)
        assert torch.equal(b_e.cost_to_go[1, 5], b_g.cost_to_go[1, 5]), it
        for name in ("cur_x", "cur_y", "arrived", "terminated", "step_counts", "state_packed"):
            assert torch.equal(getattr(sim_e, name), getattr(sim_g, name)), (it, name)
        assert sim_e.current_step == sim_g.current_step


def test_magat_stateful_graph_matches_eager():
    from iclr_2027_jointoom_amd.graphs import MagatStatefulGraph

    E, W, A = 4, 64, 96
    _, _, sim_e, _ = _setup(E, W, A, 8, density=0.3)
    _, _, sim_g, _ = _setup(E, W, A, 8, density=0.3)
    rng = np.random.default_rng(2)
    first = torch.from_numpy(rng.integers(0, 5, (E, A), dtype=np.uint8)).cuda()
    for sim in (sim_e, sim_g):
        sim.update_actions(first)
        sim.step_and_build_pyg()
    with pytest.raises(RuntimeError, match="eager step"):
        _, _, fresh, _ = _setup(E, W, A, 8, density=0.3)
        MagatStatefulGraph(fresh)
    graph = MagatStatefulGraph(sim_g)
    for it in range(5):
        acts = torch.from_numpy(rng.integers(0, 5, (E, A), dtype=np.uint8)).cuda()
        sim_e.update_actions(acts)
        sim_e.step_and_build_pyg()
        graph.actions.copy_(acts)
        graph.replay()
        torch.cuda.synchronize()
        me, mg = sim_e.memory_tensors, sim_g.memory_tensors
        for name in ("pyg_x", "pyg_pos", "edge_counts", "pyg_edge_prefix", "pyg_num_edges",
                     "goal_changed_prefix", "goal_changed_count", "changed_state_packed",
                     "cur_x", "cur_y", "state_packed"):
            assert torch.equal(me[name], mg[name]), (it, name)
        assert torch.equal(sim_e.pyg_edge_index, sim_g.pyg_edge_index), it
        assert torch.equal(sim_e.pyg_edge_attr, sim_g.pyg_edge_attr), it
        assert torch.equal(sim_e.energy_maps, sim_g.energy_maps), it
