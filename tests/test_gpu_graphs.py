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
    # pre-staged actions, one slice per replay (offsets into one allocation),
    # and an unaligned copy of one of them
    staged = torch.from_numpy(rng.integers(0, 5, (8, E, A), dtype=np.uint8)).cuda()
    odd = torch.empty(E * A + 3, dtype=torch.uint8, device="cuda")[3:].view(E, A)
    for it in range(8):
        if it == 3:
            # a changed goal: the captured build refreshes that field on the device
            for sim in (sim_e, sim_g):
                sim.goal_x[1, 5] = int(starts[1, 7, 0])
                sim.goal_y[1, 5] = int(starts[1, 7, 1])
        acts = staged[it]
        eager(sim_e, b_e, acts)
        if it in (2, 5):
            # the graph's own buffer again, after replays read other tensors
            graph.actions.copy_(acts)
            graph.replay()
        elif it == 6:
            odd.copy_(acts)
            graph.replay(odd)
        else:
            graph.replay(acts)
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
    for it in range(6):
        acts = torch.from_numpy(rng.integers(0, 5, (E, A), dtype=np.uint8)).cuda()
        sim_e.update_actions(acts)
        sim_e.step_and_build_pyg()
        if it % 3 == 1:
            graph.actions.copy_(acts)
            graph.replay()
        else:
            graph.replay(acts)
        torch.cuda.synchronize()
        me, mg = sim_e.memory_tensors, sim_g.memory_tensors
        for name in ("pyg_x", "pyg_pos", "edge_counts", "pyg_edge_prefix", "pyg_num_edges",
                     "goal_changed_prefix", "goal_changed_count", "changed_state_packed",
                     "cur_x", "cur_y", "state_packed"):
            assert torch.equal(me[name], mg[name]), (it, name)
        assert torch.equal(sim_e.pyg_edge_index, sim_g.pyg_edge_index), it
        assert torch.equal(sim_e.pyg_edge_attr, sim_g.pyg_edge_attr), it
        assert torch.equal(sim_e.energy_maps, sim_g.energy_maps), it


def test_graph_replay_rejects_mismatched_actions_before_launching():
    """replay(actions) checks the tensor before any node is retargeted or the
    graph launched: the step counter and the simulator state stay put.  A
    valid tensor of any alignment then replays."""
    from iclr_2027_jointoom_amd.graphs import MapfGPTResidentGraph

    E, W, A = 2, 32, 16
    ext, g, sim, _ = _setup(E, W, A, 5)
    b = ext.MapfGPTObservationBuilder(g, A)
    acts = torch.zeros((E, A), dtype=torch.uint8, device="cuda")
    b.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
    b.append_actions(acts)
    sim.update_actions(acts)
    sim.step_sim_only()
    graph = MapfGPTResidentGraph(sim, b)
    torch.cuda.synchronize()
    step, x = sim.current_step, sim.cur_x.clone()
    bad = [
        (acts.to(torch.int32), "uint8"),
        (torch.zeros((E, A + 1), dtype=torch.uint8, device="cuda"), "shape"),
        (torch.zeros((A, E), dtype=torch.uint8, device="cuda").t(), "contiguous"),
        (acts.cpu(), "device"),
    ]
    for t, msg in bad:
        with pytest.raises(ValueError, match=msg):
            graph.replay(t)
    torch.cuda.synchronize()
    assert sim.current_step == step
    assert torch.equal(sim.cur_x, x)
    # a source off 16-byte alignment (the capture read an aligned one): the
    # captured copy moves it byte by byte
    flat = torch.randint(0, 5, (E * A + 1,), dtype=torch.uint8, device="cuda")
    graph.replay(flat[1:].view(E, A))
    torch.cuda.synchronize()
    assert sim.current_step == step + 1
    assert torch.equal(sim.actions, flat[1:].view(E, A))
    graph.replay(acts)
    torch.cuda.synchronize()
    assert sim.current_step == step + 2
    assert torch.equal(sim.actions, acts)
