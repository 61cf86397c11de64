"""GPU parity of the CostTracer path against the CPU oracle
(oracle/costtracer.py): the environment loop of rebuttal/online-rl/
implementation/environments.py:176-219 (update_actions -> step in CostTracer
mode -> reward and goal stream -> refresh_distances -> observation, and the
episode reset from a bank), bit-exact in observations (float32), rewards,
hits, best distances, cursors, positions, goals and step counts."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _bank(seed, episodes, E, W, A, density):
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, s0, g0 = make_batch(seed, E, W, W, A, density=density)
    rng = np.random.default_rng(seed)
    pos, goal = [s0], [g0]
    for _ in range(episodes - 1):
        # other episodes: the same distinct cells, agents permuted
        p = np.stack([s0[e][rng.permutation(A)] for e in range(E)])
        g = np.stack([g0[e][rng.permutation(A)] for e in range(E)])
        pos.append(p)
        goal.append(g)
    return grids, np.stack(pos).astype(np.int16), np.stack(goal).astype(np.int16)


# 32x32 and 64x64 fields carry greedy marks in their tiles (at most 4,096
# cells); 128x128 ones hold plain distances and refresh through the
# workgroup BFS of maps of more than 64 rows
@pytest.mark.parametrize("W,E,A,horizon,steps", [(32, 3, 24, 6, 15), (64, 2, 100, 5, 11), (128, 2, 64, 5, 8)])
def test_costtracer_loop_matches_oracle(oracle, W, E, A, horizon, steps):
    from iclr_2027_jointoom_amd import profile
    from oracle.costtracer import OracleCostTracer

    print(f"[costtracer] W={W} E={E} A={A} horizon={horizon}", flush=True)
    grids, bank_pos, bank_goal = _bank(7 + A, 3, E, W, A, density=0.25)
    K = horizon + 3
    rng = np.random.default_rng(A)
    # goal streams: rolled goal sets of the bank, so every target is a free cell
    streams = np.stack([np.stack([np.roll(bank_goal[ep], k + 1, axis=1) for k in range(K)], axis=2)
                        for ep in range(3)]).astype(np.int16)  # [bank, E, A, K, 2]
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * W, 3, "costtracer", horizon)
    builder = ext.MapfGPTObservationBuilder(g, A)
    dev = "cuda"
    bp, bg = torch.from_numpy(bank_pos).to(dev), torch.from_numpy(bank_goal).to(dev)
    sbank = torch.from_numpy(streams).to(dev)
    episodes = torch.zeros(E, dtype=torch.int32, device=dev)
    env_ids = torch.arange(E, device=dev)
    stream = sbank[0].contiguous()
    cursor = torch.zeros((E, A), dtype=torch.int32, device=dev)
    best = torch.full_like(cursor, -1)
    reward = torch.empty((E, A), device=dev)
    reached = torch.empty_like(reward)
    obs = torch.empty((E, A, 2, 11, 11), device=dev)
    sim.load_state(bp[0], bg[0], torch.zeros((E, A), dtype=torch.uint8, device=dev),
                   torch.zeros(E, dtype=torch.int32, device=dev))

    ct = OracleCostTracer(grids, A, horizon)
    ct.sim.load_state(bank_pos[0], bank_goal[0])
    o_episodes = np.zeros(E, np.int64)
    o_stream = streams[0]

    def observe():
        builder.refresh_distances(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        ext.costtracer_observe(sim, builder, best, obs)
        ct.refresh_distances()
        return ct.observe()

    def compare(tag, want_obs):
        torch.cuda.synchronize()
        got = obs.cpu().numpy()
        assert np.array_equal(got, want_obs), f"{tag} obs differs at {np.argwhere(got != want_obs)[:4].tolist()}"
        assert np.array_equal(best.cpu().numpy(), ct.best), tag
        assert np.array_equal(cursor.cpu().numpy(), ct.cursor), tag
        assert np.array_equal(torch.stack((sim.cur_x, sim.cur_y), -1).cpu().numpy(), ct.sim.positions()), tag
        assert np.array_equal(torch.stack((sim.goal_x, sim.goal_y), -1).cpu().numpy(),
                              ct.goals().astype(np.int16)), tag
        assert np.array_equal(sim.step_counts.cpu().numpy(), ct.sim.step_counts), tag
        assert not any(builder.diagnostics.cpu().tolist()), tag

    compare("init", observe())
    hits = 0
    for t in range(steps):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        sim.update_actions(torch.from_numpy(acts).to(dev))
        sim.step_sim_only()
        ext.costtracer_reward_goals(sim, builder, best, stream, cursor, reward, reached)
        ct.step(acts, o_stream)
        torch.cuda.synchronize()
        assert np.array_equal(reward.cpu().numpy(), ct.rewards), t
        assert np.array_equal(reached.cpu().numpy(), ct.reached), t
        hits += int(ct.reached.sum())
        compare(f"t={t}", observe())
        if int(sim.step_counts.max()) >= horizon:
            ext.costtracer_reset(sim, bp, bg, episodes, cursor, best, episodes, horizon)
            stream = sbank[episodes.long() % bank_pos.shape[0], env_ids].contiguous()
            ct.reset_due(bank_pos, bank_goal, o_episodes, horizon)
            o_stream = streams[o_episodes % bank_pos.shape[0], np.arange(E)]
            assert episodes.cpu().tolist() == o_episodes.tolist()
            compare(f"reset t={t}", observe())
    assert int(o_episodes.sum()) >= E  # every env passed through a reset


def test_refresh_distances_matches_build_fields(oracle):
    """refresh_distances writes the same fields, rows and cache as a token build."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 2, 32, 16
    grids, starts, goals = make_batch(9, E, W, W, A)
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    b1, b2 = ext.MapfGPTObservationBuilder(g, A), ext.MapfGPTObservationBuilder(g, A)
    cx = torch.from_numpy(np.ascontiguousarray(starts[..., 0])).cuda()
    cy = torch.from_numpy(np.ascontiguousarray(starts[..., 1])).cuda()
    gx = torch.from_numpy(np.ascontiguousarray(goals[..., 0])).cuda()
    gy = torch.from_numpy(np.ascontiguousarray(goals[..., 1])).cuda()
    gx[0, 3] = 0  # an obstacle cell or not: a goal the refresh reports when it is one
    b1.refresh_distances(cx, cy, gx, gy)
    b2.build_tokens_from_state(cx, cy, gx, gy)
    torch.cuda.synchronize()
    for name in ("cost_to_go", "state_packed", "goal_cache", "labels"):
        assert torch.equal(getattr(b1, name), getattr(b2, name)), name
    d1, d2 = b1.diagnostics.cpu().tolist(), b2.diagnostics.cpu().tolist()
    assert d1[0] == d2[0] and d1[3] == d2[3] and d1[1] == 0 and d1[2] == 0
