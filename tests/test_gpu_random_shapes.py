"""Seeded random configurations across the accepted map profiles: a height
that is any multiple of 32 up to 256, a width from 8 to 256, 1 to 1,100
agents per env (at most a quarter of the cells), 1 to 3 envs, i.i.d. maps of
density 0-0.35 or mazes.  Three steps of the resident loop (token build,
history append, action copy, step) and then the stateless MAGAT build, each
against the C oracle: tokens, histories, diagnostics, positions, packed
rows, occupancy, cost_to_go, energy fields, node features and edges.  The
configurations cover every build path (single launch, two launches with
one to four row words per lane, the workgroup BFS) without naming them.
A second set runs candidate-list lifelong goals, so that builds refresh the
fields of goals changed mid-rollout on those shapes, a third the CostTracer
loop, a fourth the MAGAT stateful step with lifelong goals, a fifth both
captured loops (HIP graphs) against eager twins, and a sixth row stages
through the expert ring into both builders."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _config(seed):
    rng = np.random.default_rng(1000 + seed)
    H = 32 * int(rng.integers(1, 9))
    W = int(rng.integers(8, 257))
    kind = "maze" if rng.random() < 0.25 else "iid"
    density = float(rng.uniform(0.0, 0.35))
    A = int(rng.integers(1, max(2, min(1100, int(W * H * 0.25)))))
    E = int(rng.integers(1, 4))
    return W, H, kind, density, A, E


@pytest.mark.parametrize("seed", range(24))
def test_random_configuration_matches_oracle(oracle, seed):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions

    W, H, kind, density, A, E = _config(seed)
    tag = f"seed {seed}: {kind} {W}x{H} A{A} E{E} density {density:.2f}"
    print(tag, flush=True)
    grids, starts, goals = make_batch(seed, E, W, H, A, kind=kind, density=density)
    ext = profile(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * H, 3, "standard_mapf", 64)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    builder = ext.MapfGPTObservationBuilder(g, A)
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=64)
    osim.load_state(starts, goals)
    ob = oracle.OracleMapfGPT(grids, A)
    acts = random_actions(np.random.default_rng(seed), 3, E, A)
    for s in range(3):
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
        t = f"{tag} step {s}"
        assert np.array_equal(builder.tokens.cpu().numpy(), ob.tokens), t
        assert np.array_equal(builder.histories.cpu().numpy().view(np.uint16), ob.histories), t
        assert builder.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), t
        assert np.array_equal(torch.stack((sim.cur_x, sim.cur_y), -1).cpu().numpy(), osim.positions()), t
        assert np.array_equal(sim.state_packed.cpu().numpy().view(np.uint16), osim.state_packed), t
        assert np.array_equal(sim.grid_ocp.cpu().numpy().view(np.uint32), osim.grid_ocp), t
    assert np.array_equal(builder.cost_to_go.cpu().numpy().view(np.uint16), ob.cost_to_go), tag

    stateless = ext.StatelessGridWorldSimulator(g, A, 3)
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
    assert np.array_equal(stateless.energy_maps.cpu().numpy(), m.energy), tag
    assert np.array_equal(stateless.pyg_x.cpu().numpy(), m.pyg_x), tag
    ei, ea = m.valid_edges()
    assert np.array_equal(stateless.pyg_edge_index.cpu().numpy(), ei), tag
    assert np.array_equal(stateless.pyg_edge_attr.cpu().numpy(), ea), tag


@pytest.mark.parametrize("seed", range(12))
def test_random_lifelong_configuration_matches_oracle(oracle, seed):
    """Candidate-list lifelong goals (a third of the agents start on their
    goals) on seeded random shapes: each of six steps builds the tokens,
    refreshing the fields of the goals changed by the step before, then
    steps; tokens, diagnostics, positions, goals and cursors against the
    oracle, cost_to_go at the end."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    rng = np.random.default_rng(5000 + seed)
    H = 32 * int(rng.integers(1, 9))
    W = int(rng.integers(8, 257))
    kind = "maze" if rng.random() < 0.25 else "iid"
    density = float(rng.uniform(0.0, 0.35))
    A = int(rng.integers(1, max(2, min(1100, int(W * H * 0.2)))))
    E = int(rng.integers(1, 4))
    tag = f"seed {seed}: lifelong {kind} {W}x{H} A{A} E{E} density {density:.2f}"
    print(tag, flush=True)
    grids, starts, goals = make_batch(seed, E, W, H, A, kind=kind, density=density)
    r2 = np.random.default_rng(seed + 100)
    cells_l = [np.argwhere(gr == 0).astype(np.int16) for gr in grids]
    cells = np.full((E, max(len(c) for c in cells_l) + 3, 2), -1, np.int16)
    for e, c in enumerate(cells_l):
        cells[e, :len(c)] = r2.permutation(c)
    counts = np.array([len(c) for c in cells_l], np.int32)
    cand = r2.integers(0, 1 << 30, size=(E, A, 6)).astype(np.int32)
    goals = goals.copy()
    goals[:, ::3] = starts[:, ::3]
    ext = profile(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 2, E * W * H, 5, "lifelong", 4096)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    sim.set_goal_candidates(torch.from_numpy(cand).cuda(), torch.from_numpy(cells).cuda(),
                            torch.from_numpy(counts).cuda())
    osim = oracle.OracleSim(grids, A, task_mode=0, max_episode_steps=4096)
    osim.load_state(starts, goals)
    osim.set_goal_candidates(cand, cells, counts)
    builder = ext.MapfGPTObservationBuilder(g, A)
    ob = oracle.OracleMapfGPT(grids, A)
    acts_rng = np.random.default_rng(A + seed)
    changed = 0
    for t in range(6):
        builder.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        ob.build_state(osim.cur_x.view(np.int16), osim.cur_y.view(np.int16), osim.goal_x.view(np.int16),
                       osim.goal_y.view(np.int16))
        acts = acts_rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        if t == 0:
            acts[:] = 0
        a = torch.from_numpy(acts).cuda()
        builder.append_actions(a)
        ob.append(acts)
        sim.update_actions(a)
        sim.step_sim_only()
        osim.step(acts)
        torch.cuda.synchronize()
        tt = f"{tag} step {t}"
        assert np.array_equal(builder.tokens.cpu().numpy(), ob.tokens), tt
        assert builder.diagnostics.cpu().tolist() == ob.diagnostics.tolist(), tt
        assert np.array_equal(torch.stack((sim.cur_x, sim.cur_y), -1).cpu().numpy(), osim.positions()), tt
        assert np.array_equal(sim.goal_x.cpu().numpy(), osim.goal_x.astype(np.int16)), tt
        assert np.array_equal(sim.goal_y.cpu().numpy(), osim.goal_y.astype(np.int16)), tt
        assert np.array_equal(sim.goal_cursors.cpu().numpy(), osim.goal_cursors), tt
        changed += int(osim.goal_changed.sum())
    assert np.array_equal(builder.cost_to_go.cpu().numpy().view(np.uint16), ob.cost_to_go), tag
    assert changed >= E * len(range(0, A, 3))


@pytest.mark.parametrize("seed", range(8))
def test_random_costtracer_configuration_matches_oracle(seed):
    """The CostTracer loop (update_actions, CostTracer step, reward and goal
    stream, distance refresh, observation, horizon reset from a bank of three
    episodes) on seeded random shapes, against oracle/costtracer.py:
    observations (float32, bit for bit), rewards, hits, best distances,
    cursors, positions and step counts."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch
    from oracle.costtracer import OracleCostTracer

    r0 = np.random.default_rng(9000 + seed)
    H = 32 * int(r0.integers(1, 9))
    W = int(r0.integers(8, 257))
    density = float(r0.uniform(0.0, 0.3))
    A = int(r0.integers(1, max(2, min(600, int(W * H * 0.15)))))
    E = int(r0.integers(1, 4))
    horizon = int(r0.integers(3, 7))
    tag = f"seed {seed}: costtracer {W}x{H} A{A} E{E} density {density:.2f} horizon {horizon}"
    print(tag, flush=True)
    grids, s0, g0 = make_batch(seed, E, W, H, A, density=density)
    rng = np.random.default_rng(seed)
    pos, goal = [s0], [g0]
    for _ in range(2):  # other episodes: the same cells, agents permuted
        pos.append(np.stack([s0[e][rng.permutation(A)] for e in range(E)]))
        goal.append(np.stack([g0[e][rng.permutation(A)] for e in range(E)]))
    bank_pos, bank_goal = np.stack(pos).astype(np.int16), np.stack(goal).astype(np.int16)
    streams = np.stack([np.stack([np.roll(bank_goal[ep], k + 1, axis=1) for k in range(horizon + 3)], axis=2)
                        for ep in range(3)]).astype(np.int16)  # [bank, E, A, K, 2]
    ext = profile(W, H)
    dev = "cuda"
    g = torch.from_numpy(grids.astype(np.int32)).to(dev)
    sim = ext.GridWorldSimulator(g, A, 0, E * W * H, 3, "costtracer", horizon)
    builder = ext.MapfGPTObservationBuilder(g, A)
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

    def compare(t, want):
        torch.cuda.synchronize()
        got = obs.cpu().numpy()
        assert np.array_equal(got, want), f"{tag} {t} obs differs at {np.argwhere(got != want)[:4].tolist()}"
        assert np.array_equal(best.cpu().numpy(), ct.best), f"{tag} {t}"
        assert np.array_equal(cursor.cpu().numpy(), ct.cursor), f"{tag} {t}"
        assert np.array_equal(torch.stack((sim.cur_x, sim.cur_y), -1).cpu().numpy(), ct.sim.positions()), f"{tag} {t}"
        assert np.array_equal(sim.step_counts.cpu().numpy(), ct.sim.step_counts), f"{tag} {t}"
        assert not any(builder.diagnostics.cpu().tolist()), f"{tag} {t}"

    compare("init", observe())
    for t in range(2 * horizon + 1):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        sim.update_actions(torch.from_numpy(acts).to(dev))
        sim.step_sim_only()
        ext.costtracer_reward_goals(sim, builder, best, stream, cursor, reward, reached)
        ct.step(acts, o_stream)
        torch.cuda.synchronize()
        assert np.array_equal(reward.cpu().numpy(), ct.rewards), f"{tag} {t}"
        assert np.array_equal(reached.cpu().numpy(), ct.reached), f"{tag} {t}"
        compare(t, observe())
        if int(sim.step_counts.max()) >= horizon:
            ext.costtracer_reset(sim, bp, bg, episodes, cursor, best, episodes, horizon)
            stream = sbank[episodes.long() % 3, env_ids].contiguous()
            ct.reset_due(bank_pos, bank_goal, o_episodes, horizon)
            o_stream = streams[o_episodes % 3, np.arange(E)]
            assert episodes.cpu().tolist() == o_episodes.tolist()
            compare(f"reset {t}", observe())
    assert int(o_episodes.sum()) >= E  # every env passed through a reset


@pytest.mark.parametrize("seed", range(6))
def test_random_stateful_magat_lifelong_matches_oracle(oracle, seed):
    """The MAGAT stateful step on seeded random shapes with candidate-list
    lifelong goals: every step (step_and_build_pyg, or step_sim_only ->
    update_derived_state -> build_magat_plus_nodes ->
    finalize_magat_plus_graph) refreshes the energy fields of the goals the
    step changed, incrementally; energy fields, occupancy, node features,
    positions and edge counts, prefix and total equal a full recompute by the
    oracle after every step."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch
    from test_gpu_magat import _compare, _oracle_stateless

    r0 = np.random.default_rng(11000 + seed)
    H = 32 * int(r0.integers(1, 9))
    W = int(r0.integers(8, 257))
    density = float(r0.uniform(0.0, 0.3))
    A = int(r0.integers(1, max(2, min(1100, int(W * H * 0.15)))))
    E = int(r0.integers(1, 4))
    tag = f"seed {seed}: stateful MAGAT lifelong {W}x{H} A{A} E{E} density {density:.2f}"
    print(tag, flush=True)
    grids, starts, goals = make_batch(seed, E, W, H, A, density=density)
    r2 = np.random.default_rng(seed + 100)
    cells_l = [np.argwhere(gr == 0).astype(np.int16) for gr in grids]
    cells = np.full((E, max(len(c) for c in cells_l) + 3, 2), -1, np.int16)
    for e, c in enumerate(cells_l):
        cells[e, :len(c)] = r2.permutation(c)
    counts = np.array([len(c) for c in cells_l], np.int32)
    cand = r2.integers(0, 1 << 30, size=(E, A, 6)).astype(np.int32)
    goals = goals.copy()
    goals[:, ::3] = starts[:, ::3]
    ext = profile(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 2, E * W * H, 5, "lifelong", 4096)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    sim.set_goal_candidates(torch.from_numpy(cand).cuda(), torch.from_numpy(cells).cuda(),
                            torch.from_numpy(counts).cuda())
    osim = oracle.OracleSim(grids, A, task_mode=0, max_episode_steps=4096)
    osim.load_state(starts, goals)
    osim.set_goal_candidates(cand, cells, counts)
    rng = np.random.default_rng(seed)
    changed = 0
    for t in range(5):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        if t == 0:
            acts[:] = 0
        sim.update_actions(torch.from_numpy(acts).cuda())
        if t % 2:
            sim.step()
        else:
            sim.step_sim_only()
            sim.update_derived_state()
            sim.build_magat_plus_nodes()
            sim.finalize_magat_plus_graph()
        osim.step(acts)
        rows = osim.state_packed.copy()
        rows_reset = rows.copy()
        rows_reset[:, 7] = 1
        _compare(sim, _oracle_stateless(oracle, grids, rows_reset.view(np.int16), rows.view(np.int16)),
                 f"{tag} step {t}")
        changed += int(osim.goal_changed.sum())
    assert changed >= E * len(range(0, A, 3))


def _lifelong_pair(ext, g, grids, starts, goals, seed, E, A):
    """Two identical lifelong simulators (candidate-list goals, a third of
    the agents on their goals), for an eager run beside a graph's."""
    r2 = np.random.default_rng(seed + 100)
    cells_l = [np.argwhere(gr == 0).astype(np.int16) for gr in grids]
    cells = np.full((E, max(len(c) for c in cells_l) + 3, 2), -1, np.int16)
    for e, c in enumerate(cells_l):
        cells[e, :len(c)] = r2.permutation(c)
    counts = np.array([len(c) for c in cells_l], np.int32)
    cand = r2.integers(0, 1 << 30, size=(E, A, 6)).astype(np.int32)
    goals = goals.copy()
    goals[:, ::3] = starts[:, ::3]
    W, H = grids.shape[1:]
    sims = []
    for _ in range(2):
        sim = ext.GridWorldSimulator(g, A, 2, E * W * H, 5, "lifelong", 1 << 20)
        sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                       torch.zeros((E, A), dtype=torch.uint8, device="cuda"),
                       torch.zeros(E, dtype=torch.int32, device="cuda"))
        sim.set_goal_candidates(torch.from_numpy(cand).cuda(), torch.from_numpy(cells).cuda(),
                                torch.from_numpy(counts).cuda())
        sims.append(sim)
    return sims


@pytest.mark.parametrize("seed", range(4))
def test_random_graph_replays_match_eager(seed):
    """Both captured loops on seeded random shapes with lifelong goals (so
    captured builds and derived-state launches refresh changed goals'
    fields on the device): MapfGPTResidentGraph replays reading pre-staged
    action slices (most of them off 16-byte alignment) and
    MagatStatefulGraph replays, each against an eager twin."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.graphs import MagatStatefulGraph, MapfGPTResidentGraph
    from iclr_2027_jointoom_amd.synthetic import make_batch

    r0 = np.random.default_rng(13000 + seed)
    H = 32 * int(r0.integers(1, 9))
    W = int(r0.integers(8, 257))
    density = float(r0.uniform(0.0, 0.3))
    A = int(r0.integers(1, max(2, min(1100, int(W * H * 0.15)))))
    E = int(r0.integers(1, 4))
    tag = f"seed {seed}: graphs {W}x{H} A{A} E{E} density {density:.2f}"
    print(tag, flush=True)
    grids, starts, goals = make_batch(seed, E, W, H, A, density=density)
    ext = profile(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    rng = np.random.default_rng(seed)

    se, sg = _lifelong_pair(ext, g, grids, starts, goals, seed, E, A)
    be, bg = ext.MapfGPTObservationBuilder(g, A), ext.MapfGPTObservationBuilder(g, A)

    def eager(sim, b, acts):
        b.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        b.append_actions(acts)
        sim.update_actions(acts)
        sim.step_sim_only()

    first = torch.zeros((E, A), dtype=torch.uint8, device="cuda")
    eager(se, be, first)
    eager(sg, bg, first)
    graph = MapfGPTResidentGraph(sg, bg)
    staged = torch.from_numpy(rng.integers(0, 5, (6, E, A), dtype=np.uint8)).cuda()
    for it in range(6):
        eager(se, be, staged[it])
        graph.replay(staged[it])
        torch.cuda.synchronize()
        for name in ("tokens", "histories", "active_mask", "state_packed", "diagnostics", "goal_cache"):
            assert torch.equal(getattr(be, name), getattr(bg, name)), (tag, it, name)
        for name in ("cur_x", "cur_y", "goal_x", "goal_y", "step_counts", "state_packed"):
            assert torch.equal(getattr(se, name), getattr(sg, name)), (tag, it, name)
    assert torch.equal(be.cost_to_go, bg.cost_to_go), tag
    del graph

    se, sg = _lifelong_pair(ext, g, grids, starts, goals, seed, E, A)
    for sim in (se, sg):
        sim.update_actions(first)
        sim.step_and_build_pyg()
    graph = MagatStatefulGraph(sg)
    for it in range(5):
        acts = torch.from_numpy(rng.integers(0, 5, (E, A), dtype=np.uint8)).cuda()
        se.update_actions(acts)
        se.step_and_build_pyg()
        graph.replay(acts)
        torch.cuda.synchronize()
        me, mg = se.memory_tensors, sg.memory_tensors
        for name in ("pyg_x", "pyg_pos", "edge_counts", "pyg_edge_prefix", "pyg_num_edges",
                     "goal_changed_prefix", "goal_changed_count", "changed_state_packed",
                     "cur_x", "cur_y", "state_packed"):
            assert torch.equal(me[name], mg[name]), (tag, it, name)
        assert torch.equal(se.pyg_edge_index, sg.pyg_edge_index), (tag, it)
        assert torch.equal(se.pyg_edge_attr, sg.pyg_edge_attr), (tag, it)
        assert torch.equal(se.energy_maps, sg.energy_maps), (tag, it)


@pytest.mark.parametrize("seed", range(3))
def test_random_ring_stages_match_oracle(oracle, seed):
    """Row stages on seeded random shapes through the expert ring (producer
    threads -> shared ring -> pinned staging -> HBM ring of 2-4 stage
    slots): 13-column stages into MapfGPTOnlinePipeline's builder (tokens)
    and 8-column stages into ExtremeMAPFPipeline's MAGAT simulator (node
    features and edges), against the oracle fed the same rows."""
    import time

    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.ring import ExtremeMAPFPipeline, MapfGPTOnlinePipeline
    from iclr_2027_jointoom_amd.synthetic import make_batch
    from test_gpu_ring import _TokenRuntime, _produce

    r0 = np.random.default_rng(15000 + seed)
    H = 32 * int(r0.integers(1, 9))
    W = int(r0.integers(8, 257))
    A = int(r0.integers(1, max(2, min(700, int(W * H * 0.15)))))
    E = int(r0.integers(1, 5))
    S = int(r0.integers(2, 6))
    slots = int(r0.integers(2, 5))
    tag = f"seed {seed}: ring {W}x{H} A{A} E{E} stages {S} slots {slots}"
    print(tag, flush=True)

    def stages_for(features, s_seed):
        grids, starts, goals = make_batch(s_seed, E, W, H, A)
        rng = np.random.default_rng(s_seed)
        stages = np.zeros((S, E * A, features), np.uint16)
        pos = starts.astype(np.int64)
        for s in range(S):
            blk = stages[s].reshape(E, A, features)
            blk[:, :, 0] = np.arange(E)[:, None]
            blk[:, :, 1] = np.arange(A)[None]
            blk[:, :, 2:4] = pos
            blk[:, :, 4:6] = goals
            blk[:, :, 6] = rng.integers(0, 5, size=(E, A))
            blk[:, :, 7] = 1 if s == 0 else (rng.random((E, A)) < 0.05)
            if features == 13:
                blk[:, :, 8:13] = rng.integers(0, 6, size=(E, A, 5))
            pos = np.roll(pos, 1, axis=1)  # distinct cells, still on the free component
        return grids, stages

    grids, stages = stages_for(13, seed)
    builder = profile(W, H).MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)
    runtime = _TokenRuntime()
    pipe = MapfGPTOnlinePipeline(builder, runtime, capacity=slots * E * A, batch_threshold=E * A).initialize()
    pipe.dma_worker_loop()
    threads = _produce(pipe.ring_buffer, stages, E, A)
    deadline = time.monotonic() + 60
    try:
        while len(runtime.tokens) < S:
            if pipe.consume_once() is None:
                assert time.monotonic() < deadline, (tag, pipe.get_stats())
                time.sleep(0.0005)
    finally:
        pipe.shutdown()
    for t in threads:
        t.join(timeout=5)
    ob = oracle.OracleMapfGPT(grids, A)
    for s in range(S):
        ob.build_rows(stages[s])
        assert np.array_equal(runtime.tokens[s].cpu().numpy(), ob.tokens), (tag, s)

    grids, stages = stages_for(8, seed + 1)
    sim = profile(W, H).StatelessGridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 3)
    pipe = ExtremeMAPFPipeline(sim, capacity=slots * E * A, batch_threshold=E * A).initialize()
    pipe.dma_worker_loop()
    threads = _produce(pipe.ring_buffer, stages, E, A)
    m = oracle.OracleMagat(grids, A)
    deadline = time.monotonic() + 60
    try:
        for s in range(S):
            x = None
            while x is None:
                x = pipe.train_step()
                if x is None:
                    assert time.monotonic() < deadline, (tag, pipe.get_stats())
                    time.sleep(0.0005)
            sim.materialize_pyg_inputs()
            rows = stages[s]
            reset = rows[rows[:, 7] != 0]
            m.update_energy(reset, len(reset))
            m.refresh(rows)
            m.nodes()
            m.edges()
            torch.cuda.synchronize()
            assert np.array_equal(sim.pyg_x.cpu().numpy(), m.pyg_x), (tag, s)
            assert np.array_equal(sim.pyg_edge_index.cpu().numpy(), m.valid_edges()[0]), (tag, s)
    finally:
        pipe.shutdown()
    for t in threads:
        t.join(timeout=5)
