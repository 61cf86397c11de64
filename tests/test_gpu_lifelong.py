"""GPU parity of the deterministic lifelong goal assignment (set_goal_candidates,
canonical agent order) and of the CostTracer step mode against the C oracle
(rebuttal/online-rl/native/src/cuda_backend/128_agents_map_step.cu:219-222,
303-330; grid_world_simulator.cpp:901-918).  Bit-exact: positions, goals,
cursors, goal-changed flags, rewards, occupancy, packed rows, step counts."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from test_gpu_step import compare_with_oracle  # noqa: E402


def _candidate_setup(seed, E, W, A, K=6, on_goal_every=3, density=0.2):
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(seed, E, W, W, A, density=density)
    rng = np.random.default_rng(seed + 100)
    cells_l = [np.argwhere(g == 0).astype(np.int16) for g in grids]
    stride = max(len(c) for c in cells_l) + 3  # padded rows past the counts are never read
    cells = np.full((E, stride, 2), -1, np.int16)
    for e, c in enumerate(cells_l):
        cells[e, :len(c)] = rng.permutation(c)
    counts = np.array([len(c) for c in cells_l], np.int32)
    candidates = rng.integers(0, 1 << 30, size=(E, A, K)).astype(np.int32)
    goals = goals.copy()
    goals[:, ::on_goal_every] = starts[:, ::on_goal_every]
    return grids, starts, goals, cells, counts, candidates


def _compare_lifelong(sim, osim, tag):
    compare_with_oracle(sim, osim, tag)
    for name, got, exp in (("goal_x", sim.goal_x, osim.goal_x.astype(np.int16)),
                           ("goal_y", sim.goal_y, osim.goal_y.astype(np.int16)),
                           ("goal_cursors", sim.goal_cursors, osim.goal_cursors)):
        g = got.cpu().numpy()
        assert np.array_equal(g, exp), f"{tag} {name} differs at {np.argwhere(g != exp)[:5].tolist()}"


@pytest.mark.parametrize("W,E,A,T", [(32, 3, 40, 30), (64, 4, 128, 25), (64, 2, 700, 12), (128, 2, 300, 10)])
def test_candidate_lifelong_rollouts_match_oracle(oracle, W, E, A, T):
    from iclr_2027_jointoom_amd import profile

    print(f"[lifelong] W={W} E={E} A={A} T={T}", flush=True)
    grids, starts, goals, cells, counts, candidates = _candidate_setup(11 + A, E, W, A)
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 2, E * W * W, 5, "lifelong", 4096)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    sim.set_goal_candidates(torch.from_numpy(candidates).cuda(), torch.from_numpy(cells).cuda(),
                            torch.from_numpy(counts).cuda())
    osim = oracle.OracleSim(grids, A, task_mode=0, max_episode_steps=4096)
    osim.load_state(starts, goals)
    osim.set_goal_candidates(candidates, cells, counts)
    rng = np.random.default_rng(A)
    changed = 0
    for t in range(T):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        if t == 0:
            acts[:] = 0
        sim.update_actions(torch.from_numpy(acts).cuda())
        sim.step_sim_only()
        osim.step(acts)
        _compare_lifelong(sim, osim, f"t={t}")
        changed += int(osim.goal_changed.sum())
    assert changed >= E * len(range(0, A, 3))


def test_set_goal_candidates_contract():
    from iclr_2027_jointoom_amd import profile

    ext = profile(32, 32)
    E, A = 2, 4
    g = torch.zeros((E, 32, 32), dtype=torch.int32, device="cuda")
    sim = ext.GridWorldSimulator(g, A, 2, E * 1024, 5, "lifelong", 64)
    cand = torch.zeros((E, A, 3), dtype=torch.int32, device="cuda")
    cells = torch.zeros((E, 10, 2), dtype=torch.int16, device="cuda")
    counts = torch.full((E,), 8, dtype=torch.int32, device="cuda")
    cases = [
        ((cand.cpu(), cells, counts), "must be CUDA"),
        ((cand.to(torch.int64), cells, counts), "dtype mismatch"),
        ((cand[:, :2], cells, counts), r"\[N,A,K\]"),
        ((cand, cells[:, :, :1], counts), r"\[N,F,2\]"),
        ((cand, cells, torch.full((E,), A, dtype=torch.int32, device="cuda")), "invalid free-cell counts"),
        ((cand, cells, torch.full((E,), 11, dtype=torch.int32, device="cuda")), "invalid free-cell counts"),
    ]
    for args, msg in cases:
        with pytest.raises(RuntimeError, match=msg):
            sim.set_goal_candidates(*args)
    assert sim.goal_cursors is None
    sim.set_goal_candidates(cand, cells, counts)
    assert sim.goal_cursors.shape == (E, A) and sim.goal_cursors.dtype == torch.int32
    assert int(sim.goal_cursors.abs().sum()) == 0


@pytest.mark.parametrize("W,E,A", [(32, 3, 50), (64, 2, 300)])
def test_costtracer_mode_matches_oracle(oracle, W, E, A):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    print(f"[costtracer step] W={W} E={E} A={A}", flush=True)
    grids, starts, goals = make_batch(3 + A, E, W, W, A)
    ext = profile(W, W)
    sim = ext.GridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 2, E * W * W, 5,
                                 "costtracer", 64)
    assert sim.task_mode == "costtracer"
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                   torch.zeros(E, dtype=torch.int32, device="cuda"))
    osim = oracle.OracleSim(grids, A, task_mode=2, max_episode_steps=64)
    osim.load_state(starts, goals)
    rng = np.random.default_rng(1)
    for t in range(8):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        sim.update_actions(torch.from_numpy(acts).cuda())
        sim.step_sim_only()
        osim.step(acts)
        compare_with_oracle(sim, osim, f"t={t}")
    assert sim.step_counts.cpu().tolist() == [8] * E


# (252, 256, 3, 1199): four agents per thread, and step tables with the
# half-full hash that come within 256 bytes of the 160 KB of LDS (the
# kernel's own reduction buffer): they now take the fuller hash, where that
# launch had run past the LDS
@pytest.mark.parametrize("W,H,E,A,T,extent", [(32, 32, 3, 40, 40, None), (64, 64, 4, 128, 30, (50, 60)),
                                              (96, 96, 2, 300, 20, (65, 65)), (128, 128, 2, 500, 12, None),
                                              (252, 256, 3, 1199, 6, None)])
def test_random_lifelong_rollouts_match_oracle(oracle, W, H, E, A, T, extent):
    """The generator-drawn lifelong path (the default task mode without
    candidate lists; 128_agents_map_step.cu:265-343 and
    grid_world_cuda.cu:225-479 with cuRAND's racing draws replaced by
    per-agent xorshift64* draws settled in id order): init_rng, the free-cell
    lists inside the real extents, the random distinct starts and goals, then
    a reload with a third of the agents on their goal and a rollout in which
    every agent reaching its goal draws a new one.  Cells, goals, flags, packed
    rows, occupancy and every generator state equal the oracle's after each
    step."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import iid_grid

    print(f"[random lifelong] {W}x{H} E={E} A={A} T={T} extent={extent}", flush=True)
    rng = np.random.default_rng(W + A)
    grids = np.stack([iid_grid(rng, W, H, 0.2) for _ in range(E)])
    extents = np.tile([W, H] if extent is None else extent, (E, 1)).astype(np.int32)
    ext = profile(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    seed = 4242 + A
    sim = ext.GridWorldSimulator(g, A, 2, E * W * H, seed)
    sim.set_real_map_extents(torch.from_numpy(extents).cuda())
    sim.run_initialization()
    osim = oracle.OracleSim(grids, A, task_mode=0, max_episode_steps=256)
    osim.seed_rng(seed)
    osim.lifelong_init(extents)
    torch.cuda.synchronize()
    assert np.array_equal(sim.counts.cpu().numpy(), osim.env_counts)
    assert np.array_equal(sim.memory_tensors["offsets"].cpu().numpy(), osim.env_offsets)
    fc = sim.memory_tensors["free_cell_list"].cpu().numpy().view(np.uint32)
    for e in range(E):
        lo = e * W * H
        assert np.array_equal(fc[lo:lo + osim.env_counts[e]], osim.free_cells[lo:lo + osim.env_counts[e]])

    def check(tag):
        _compare_lifelong_goals(sim, osim, E * A, tag)

    check("init")
    # reload: every third agent's goal on its start, so it draws at once
    starts = osim.positions()
    goals = np.stack([osim.goal_x, osim.goal_y], -1).astype(np.int16)
    goals[:, ::3] = starts[:, ::3]
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    osim.load_state(starts, goals)
    changed = 0
    for t in range(T):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        if t == 0:
            acts[:] = 0
        sim.update_actions(torch.from_numpy(acts).cuda())
        sim.step_sim_only()
        osim.step(acts)
        compare_with_oracle(sim, osim, f"step {t}")
        check(f"step {t}")
        changed += int(osim.goal_changed.sum())
    assert changed >= E * len(range(0, A, 3))


def test_random_lifelong_draws_past_held_goals_match_oracle(oracle):
    """Seven agents in a 4 x 4 real extent of free cells: most cells of the
    free-cell list are goals held by agents off their goal, so a draw often
    finds its first two cells held and reads further cells of the list
    (the settling thread's fallback).  Every agent starts on its goal, so all
    draw at once, in id order, at the first step.  Cells, goals and
    generator states equal the oracle's after each step."""
    from iclr_2027_jointoom_amd import profile

    W = H = 32
    E, A, T = 3, 7, 60
    grids = np.zeros((E, W, H), np.uint8)
    extents = np.tile([4, 4], (E, 1)).astype(np.int32)
    ext = profile(W, H)
    seed = 777
    sim = ext.GridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 2, E * W * H, seed)
    sim.set_real_map_extents(torch.from_numpy(extents).cuda())
    sim.run_initialization()
    osim = oracle.OracleSim(grids, A, task_mode=0, max_episode_steps=256)
    osim.seed_rng(seed)
    osim.lifelong_init(extents)
    _compare_lifelong_goals(sim, osim, E * A, "init")
    starts = osim.positions()
    goals = starts.astype(np.int16)  # every agent on its goal
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    osim.load_state(starts, goals)
    rng = np.random.default_rng(5)
    changed = 0
    for t in range(T):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        if t == 0:
            acts[:] = 0
        sim.update_actions(torch.from_numpy(acts).cuda())
        sim.step_sim_only()
        osim.step(acts)
        compare_with_oracle(sim, osim, f"step {t}")
        _compare_lifelong_goals(sim, osim, E * A, f"step {t}")
        changed += int(osim.goal_changed.sum())
    assert changed >= E * A


def _compare_lifelong_goals(sim, osim, n, tag):
    torch.cuda.synchronize()
    for name, got, exp in (("cur_x", sim.cur_x, osim.cur_x.astype(np.int16)),
                           ("cur_y", sim.cur_y, osim.cur_y.astype(np.int16)),
                           ("goal_x", sim.goal_x, osim.goal_x.astype(np.int16)),
                           ("goal_y", sim.goal_y, osim.goal_y.astype(np.int16)),
                           ("rng_states", sim.memory_tensors["rng_states"][:n], osim.rng_state.view(np.int64))):
        g = got.cpu().numpy()
        assert np.array_equal(g, exp), f"{tag} {name} differs at {np.argwhere(g != exp)[:5].tolist()}"
