"""GPU parity of the batched step (jl_step / jl_load_state) against the C oracle.

Ports the KATs of /root/reference/tests/expert/test_stateful_standard_mapf.py
and test_transition_adapters.py:884-1027 to the gfx950 path.  Bit-exact:
positions, outcomes, arrival, done flags, step counts, occupancy, rewards
and packed rows.
"""
import json
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
FIELDS = {1: "wall_rejections", 2: "vertex_rejections", 3: "edge_swap_rejections", 4: "chain_rejections"}


def ext_for(w, h):
    from iclr_2027_jointoom_amd import profile

    return profile(w, h)


def _sim(ext, *, num_envs=1, num_agents=1, seed=7, task_mode=None, max_episode_steps=256):
    grid = torch.zeros((num_envs, ext.COMPILED_MAP_W, ext.COMPILED_MAP_H), dtype=torch.int32, device="cuda")
    args = [grid, num_agents, 2, num_envs * ext.COMPILED_MAP_W * ext.COMPILED_MAP_H, seed]
    if task_mode is not None:
        args.extend([task_mode, max_episode_steps])
    return ext.GridWorldSimulator(*args)


def _load(sim, positions, goals, *, arrived=None, step_counts=None):
    positions = torch.tensor(positions, dtype=torch.int16, device="cuda").contiguous()
    goals = torch.tensor(goals, dtype=torch.int16, device="cuda").contiguous()
    E, A, _ = positions.shape
    arrived = torch.tensor(arrived if arrived is not None else [[0] * A] * E, dtype=torch.uint8, device="cuda")
    counts = torch.tensor(step_counts if step_counts is not None else [0] * E, dtype=torch.int32, device="cuda")
    sim.load_state(positions, goals, arrived.contiguous(), counts.contiguous())
    torch.cuda.synchronize()


def _act(sim, actions):
    sim.update_actions(torch.tensor(actions, dtype=torch.uint8, device="cuda").contiguous())


def compare_with_oracle(sim, osim, tag=""):
    torch.cuda.synchronize()
    pairs = [
        ("cur_x", sim.cur_x, osim.cur_x.astype(np.int16)),
        ("cur_y", sim.cur_y, osim.cur_y.astype(np.int16)),
        ("outcomes", sim.outcomes, osim.outcomes),
        ("arrived", sim.arrived, osim.arrived),
        ("terminated", sim.terminated, osim.terminated),
        ("truncated", sim.truncated, osim.truncated),
        ("step_counts", sim.step_counts, osim.step_counts),
        ("rewards", sim.rewards, osim.rewards),
        ("grid_ocp", sim.grid_ocp, osim.grid_ocp.view(np.int32)),
        ("state_packed", sim.state_packed, osim.state_packed.view(np.int16)),
        ("goal_changed", sim.goal_changed_flags, osim.goal_changed),
    ]
    for name, got, exp in pairs:
        g = got.cpu().numpy()
        assert np.array_equal(g, exp), f"{tag} {name} differs at {np.argwhere(g != exp)[:5].tolist()}"


@pytest.mark.parametrize("name", list(json.loads((GOLDEN / "directed_fixtures.json").read_text())["cases"]))
def test_directed_fixtures_gpu(name):
    data = json.loads((GOLDEN / "directed_fixtures.json").read_text())
    case = data["cases"][name]
    ext = ext_for(128, 128)
    A = len(case["actions"])
    grid = torch.zeros((1, 128, 128), dtype=torch.int32, device="cuda")
    for x, y in case.get("walls", []):
        grid[0, x, y] = 1
    sim = ext.GridWorldSimulator(grid, A, 0, 128 * 128, 7, "standard_mapf", 1)
    arrived = [[int(v) for v in case.get("arrived", [False] * A)]]
    _load(sim, [case["positions"]], [case["goals"]], arrived=arrived)
    _act(sim, [case["actions"]])
    sim.step_sim_only()
    torch.cuda.synchronize()
    pos = torch.stack([sim.cur_x, sim.cur_y], -1).cpu().tolist()
    assert pos == [case["expected"]]
    assert sim.terminated.bool().cpu().tolist() == case.get("terminated", [False])
    assert sim.truncated.bool().cpu().tolist() == case.get("truncated", [True])
    assert sim.step_counts.cpu().tolist() == [1]
    out = sim.outcomes.cpu().numpy()
    for c, field in FIELDS.items():
        assert int((out == c).sum()) == case["collision"].get(field, 0), field


def test_c1_plumbing_rollout_matches_oracle_every_step(oracle):
    """C1: 1 env, 32x32 p=0.2, 64 agents, 128 random steps: step + tokens each step."""
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions

    grids, starts, goals = make_batch(20260728, 1, 32, 32, 64)
    actions = random_actions(np.random.default_rng(1), 128, 1, 64)
    ext = ext_for(32, 32)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, 64, 0, 32 * 32, 7, "standard_mapf", 128)
    sim.load_state(
        torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
        torch.zeros((1, 64), dtype=torch.uint8, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda"),
    )
    builder = ext.MapfGPTObservationBuilder(g, 64)
    builder.reset_histories()
    osim = oracle.OracleSim(grids, 64, task_mode=1, max_episode_steps=128)
    osim.load_state(starts, goals)
    ob = oracle.OracleMapfGPT(grids, 64)
    compare_with_oracle(sim, osim, "load")
    for step in range(128):
        builder.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        ob.build_state(osim.cur_x.view(np.int16), osim.cur_y.view(np.int16),
                       osim.goal_x.view(np.int16), osim.goal_y.view(np.int16))
        torch.cuda.synchronize()
        assert np.array_equal(builder.tokens.cpu().numpy(), ob.tokens), f"tokens step {step}"
        assert np.array_equal(builder.active_mask.cpu().numpy().astype(np.uint8), ob.active_mask)
        assert builder.diagnostics.cpu().tolist() == ob.diagnostics.tolist() == [0, 0, 0, 0]
        a = torch.from_numpy(actions[step]).cuda()
        builder.append_actions(a)
        ob.append(actions[step])
        sim.update_actions(a)
        sim.step_sim_only()
        osim.step(actions[step])
        compare_with_oracle(sim, osim, f"step {step}")
        assert np.array_equal(builder.histories.cpu().numpy(), ob.histories.view(np.int16))


@pytest.mark.parametrize("W,H,E,A", [(64, 64, 64, 128), (128, 128, 8, 512), (256, 256, 2, 1024),
                                     (128, 128, 2, 1100)])
def test_random_rollouts_match_oracle(oracle, W, H, E, A):
    """One thread per agent up to 1,024 agents per env, four per thread beyond."""
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions

    grids, starts, goals = make_batch(W + A, E, W, H, A)
    actions = random_actions(np.random.default_rng(W), 24, E, A)
    ext = ext_for(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * H, 7, "standard_mapf", 20)
    sim.load_state(
        torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
        torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"),
    )
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=20)
    osim.load_state(starts, goals)
    for step in range(24):  # runs past the horizon: done envs must freeze
        sim.update_actions(torch.from_numpy(actions[step]).cuda())
        sim.step_sim_only()
        osim.step(actions[step])
        compare_with_oracle(sim, osim, f"step {step}")


def test_dense_conflicts_match_oracle(oracle):
    """Crowded open map: long chains, cycles, swaps and vertex ties every step."""
    E, W, H, A = 16, 32, 32, 600
    rng = np.random.default_rng(77)
    grids = np.zeros((E, W, H), np.uint8)
    starts = np.stack([np.stack(np.divmod(rng.choice(W * H, A, replace=False), H), -1) for _ in range(E)]).astype(np.int16)
    goals = np.stack([np.stack(np.divmod(rng.choice(W * H, A, replace=False), H), -1) for _ in range(E)]).astype(np.int16)
    ext = ext_for(W, H)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * H, 7, "standard_mapf", 1000)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=1000)
    osim.load_state(starts, goals)
    for step in range(16):
        acts = rng.integers(0, 5, size=(E, A), dtype=np.uint8)
        sim.update_actions(torch.from_numpy(acts).cuda())
        sim.step_sim_only()
        osim.step(acts)
        compare_with_oracle(sim, osim, f"step {step}")


# ---- API KATs ported from test_stateful_standard_mapf.py -----------------

def test_mode_properties_and_validation():
    ext = ext_for(128, 128)
    sim = _sim(ext)
    assert sim.task_mode == "lifelong" and sim.max_episode_steps == 256
    with pytest.raises(AttributeError):
        sim.task_mode = "standard_mapf"
    sim = _sim(ext, task_mode="standard_mapf", max_episode_steps=17)
    assert sim.task_mode == "standard_mapf" and sim.max_episode_steps == 17
    for name in ("arrived", "terminated", "truncated", "step_counts"):
        value = getattr(sim, name)
        with pytest.raises(AttributeError):
            setattr(sim, name, value.clone())
        assert getattr(sim, name) is value
    with pytest.raises((RuntimeError, ValueError), match="Unknown task mode"):
        _sim(ext, task_mode="not-a-mapf-mode")
    with pytest.raises((RuntimeError, ValueError), match="positive"):
        _sim(ext, task_mode="standard_mapf", max_episode_steps=0)


@pytest.mark.parametrize(
    ("positions", "goals", "arrived", "step_counts", "message"),
    [
        ([[[-1, 2]]], [[[3, 4]]], [[0]], [0], "bounds"),
        ([[[2, 2]]], [[[128, 4]]], [[0]], [0], "bounds"),
        ([[[2, 2]]], [[[3, 4]]], [[1]], [0], "arrived agents"),
        ([[[2, 2]]], [[[3, 4]]], [[0]], [-1], "step_counts"),
        ([[[2, 2]]], [[[3, 4]]], [[0]], [257], "step_counts"),
    ],
)
def test_load_state_validates(positions, goals, arrived, step_counts, message):
    sim = _sim(ext_for(128, 128), task_mode="standard_mapf")
    with pytest.raises(RuntimeError, match=message):
        _load(sim, positions, goals, arrived=arrived, step_counts=step_counts)


@pytest.mark.parametrize(("make", "message"), [
    (lambda a: a.to(torch.int16), "new_actions must be uint8"),
    (lambda a: a.cpu(), "new_actions must be CUDA"),
    (lambda a: a[:, :1].contiguous(), "new_actions shape mismatch"),
    (lambda a: torch.zeros((2, 4), dtype=torch.uint8, device="cuda")[:, ::2], "new_actions must be contiguous"),
])
def test_update_actions_validates(make, message):
    """update_actions keeps the reference's checks and messages
    (grid_world_simulator.cpp:678-688) behind its one-test fast path."""
    sim = _sim(ext_for(128, 128), num_envs=2, num_agents=2, task_mode="standard_mapf")
    good = torch.zeros((2, 2), dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match=message):
        sim.update_actions(make(good))
    sim.update_actions(good)


@pytest.mark.parametrize("field", [0, 1, 2, 3])
@pytest.mark.parametrize(("violation", "message"), [
    ("cpu", "must be CUDA"), ("dtype", "must be (int16|uint8|int32)"),
    ("shape", "must have shape"), ("noncontiguous", "must be contiguous")])
def test_load_state_tensor_contract(field, violation, message):
    sim = _sim(ext_for(128, 128), num_envs=2, num_agents=2, task_mode="standard_mapf")
    tensors = [
        torch.tensor([[[2, 3], [3, 4]], [[4, 5], [5, 6]]], dtype=torch.int16, device="cuda"),
        torch.tensor([[[20, 21], [21, 22]], [[22, 23], [23, 24]]], dtype=torch.int16, device="cuda"),
        torch.zeros((2, 2), dtype=torch.uint8, device="cuda"),
        torch.zeros((2,), dtype=torch.int32, device="cuda"),
    ]
    original = tensors[field]
    if violation == "cpu":
        bad = original.cpu()
    elif violation == "dtype":
        bad = original.to(torch.int64)
    elif violation == "shape":
        bad = original.unsqueeze(-1)
    else:
        backing = torch.zeros(original.shape[:-1] + (original.shape[-1] * 2,), dtype=original.dtype, device="cuda")
        bad = backing[..., ::2]
        bad.copy_(original)
        assert not bad.is_contiguous()
    tensors[field] = bad
    with pytest.raises(RuntimeError, match=message):
        sim.load_state(*tensors)
    tensors[field] = original
    tensors[2] = torch.zeros((2, 2), dtype=torch.uint8, device="cuda")
    tensors[2][1, 1] = 2
    with pytest.raises(RuntimeError, match="arrived values must be 0 or 1"):
        sim.load_state(*tensors)


def test_load_state_layout_and_packed_rows():
    sim = _sim(ext_for(128, 128), num_envs=2, num_agents=2, task_mode="standard_mapf")
    positions = [[[2, 3], [4, 35]], [[7, 8], [9, 10]]]
    goals = [[[2, 3], [6, 7]], [[11, 12], [13, 14]]]
    _load(sim, positions, goals, arrived=[[1, 0], [0, 0]], step_counts=[3, 4])
    assert sim.cur_x.cpu().tolist() == [[2, 4], [7, 9]]
    assert sim.cur_y.cpu().tolist() == [[3, 35], [8, 10]]
    assert sim.step_counts.cpu().tolist() == [3, 4]
    assert bool(sim.goal_changed_flags.all())
    expected = torch.zeros((2, 512), dtype=torch.int64)
    for e, env in enumerate(positions):
        for x, y in env:
            expected[e, x * 4 + (y >> 5)] |= 1 << (y & 31)
    assert torch.equal(sim.grid_ocp.cpu().to(torch.int64) & 0xFFFFFFFF, expected & 0xFFFFFFFF)
    assert sim.state_packed.cpu().tolist() == [
        [0, 0, 2, 3, 2, 3, 0, 1], [0, 1, 4, 35, 6, 7, 0, 1],
        [1, 0, 7, 8, 11, 12, 0, 1], [1, 1, 9, 10, 13, 14, 0, 1]]


def test_update_actions_copies_and_load_state_resets_actions():
    ext = ext_for(128, 128)
    sim = _sim(ext, task_mode="standard_mapf")
    _load(sim, [[[10, 10]]], [[[20, 20]]])
    caller = torch.tensor([[2]], dtype=torch.uint8, device="cuda")
    sim.update_actions(caller)
    caller.zero_()
    sim.step_sim_only()
    torch.cuda.synchronize()
    assert sim.cur_x.cpu().tolist() == [[11]]
    _load(sim, [[[30, 30]]], [[[40, 40]]])
    sim.step_sim_only()
    torch.cuda.synchronize()
    assert sim.cur_x.cpu().tolist() == [[30]] and sim.state_packed[:, 6].cpu().tolist() == [0]
    sim2 = _sim(ext, num_agents=2, task_mode="standard_mapf")
    with pytest.raises(RuntimeError, match="CUDA"):
        sim2.update_actions(torch.zeros((1, 2), dtype=torch.uint8))
    backing = torch.zeros((1, 4), dtype=torch.uint8, device="cuda")
    noncontiguous = backing[:, ::2]
    assert not noncontiguous.is_contiguous()
    with pytest.raises(RuntimeError, match="contiguous"):
        sim2.update_actions(noncontiguous)


@pytest.mark.parametrize("E,A,offset", [(3, 37, 0), (3, 37, 1), (4, 64, 0), (2, 8, 5)])
def test_update_actions_copies_every_byte(E, A, offset):
    """Aligned sources take 16-byte words plus a byte tail, misaligned ones bytes."""
    ext = ext_for(32, 32)
    sim = _sim(ext, num_envs=E, num_agents=A, task_mode="standard_mapf")
    backing = torch.randint(0, 256, (E * A + 16,), dtype=torch.uint8, device="cuda")
    src = backing[offset:offset + E * A].view(E, A)
    assert src.is_contiguous()
    sim.actions.fill_(255)
    sim.update_actions(src)
    torch.cuda.synchronize()
    assert torch.equal(sim.actions, src)


def test_done_env_freezes_and_arrival_kats():
    ext = ext_for(128, 128)
    sim = _sim(ext, num_agents=2, task_mode="standard_mapf")
    _load(sim, [[[10, 10], [20, 20]]], [[[10, 10], [30, 30]]], arrived=[[1, 0]])
    _act(sim, [[2, 0]])
    sim.step_sim_only()
    torch.cuda.synchronize()
    assert sim.cur_x.cpu().tolist() == [[10, 20]] and sim.state_packed[:, 6].cpu().tolist() == [0, 0]
    for kind in ("terminated", "truncated"):
        if kind == "terminated":
            sim = _sim(ext, task_mode="standard_mapf")
            _load(sim, [[[10, 10]]], [[[11, 10]]])
            _act(sim, [[2]])
        else:
            sim = _sim(ext, task_mode="standard_mapf", max_episode_steps=1)
            _load(sim, [[[10, 10]]], [[[20, 20]]])
            _act(sim, [[0]])
        sim.step_sim_only()
        torch.cuda.synchronize()
        before = [t.clone() for t in (sim.cur_x, sim.cur_y, sim.step_counts, sim.state_packed, sim.grid_ocp)]
        _act(sim, [[2]])
        sim.step_sim_only()
        torch.cuda.synchronize()
        after = (sim.cur_x, sim.cur_y, sim.step_counts, sim.state_packed, sim.grid_ocp)
        assert all(torch.equal(a, b) for a, b in zip(before, after))


def test_nondefault_stream_orders_load_actions_and_step():
    sim = _sim(ext_for(128, 128), task_mode="standard_mapf")
    stream = torch.cuda.Stream()
    positions = torch.tensor([[[10, 10]]], dtype=torch.int16, device="cuda")
    goals = torch.tensor([[[20, 20]]], dtype=torch.int16, device="cuda")
    arrived = torch.zeros((1, 1), dtype=torch.uint8, device="cuda")
    counts = torch.zeros((1,), dtype=torch.int32, device="cuda")
    actions = torch.tensor([[2]], dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        sim.load_state(positions, goals, arrived, counts)
        sim.update_actions(actions)
        sim.step_sim_only()
    stream.synchronize()
    assert sim.cur_x.cpu().tolist() == [[11]] and sim.step_counts.cpu().tolist() == [1]


def test_lifelong_initialization_and_goal_reassignment():
    """Lifelong mode: distinct free starts/goals; an agent on its goal draws a
    new free goal.  The reference's exact cell for seed 7, (46, 39)
    (test_stateful_standard_mapf.py:517-529), comes from cuRAND's XORWOW
    stream, which is not reproduced: parity unpinned for the drawn cell."""
    ext = ext_for(128, 128)
    grid = torch.zeros((2, 128, 128), dtype=torch.int32, device="cuda")
    grid[:, 0:4, :] = 1
    sim = ext.GridWorldSimulator(grid, 8, 2, 2 * 128 * 128, 7)
    sim.run_initialization()
    torch.cuda.synchronize()
    starts = torch.stack([sim.cur_x, sim.cur_y], -1).cpu().numpy()
    goals = torch.stack([sim.goal_x, sim.goal_y], -1).cpu().numpy()
    for e in range(2):
        cells = np.concatenate([starts[e], goals[e]])
        assert len({tuple(c) for c in cells}) == 16
        assert np.all(cells[:, 0] >= 4)
    assert sim.counts.cpu().tolist() == [124 * 128] * 2
    sim.cur_x[0, 0] = 10
    sim.cur_y[0, 0] = 10
    sim.goal_x[0, 0] = 10
    sim.goal_y[0, 0] = 10
    _act(sim, [[0] * 8, [0] * 8])
    sim.step_sim_only()
    torch.cuda.synchronize()
    new = (int(sim.goal_x[0, 0]), int(sim.goal_y[0, 0]))
    assert new != (10, 10) and new[0] >= 4
    assert sim.goal_changed_flags.cpu()[0].tolist() == [1] + [0] * 7
    assert sim.state_packed[0].cpu().tolist() == [0, 0, 10, 10, new[0], new[1], 0, 1]


def test_c2_full_size_invariants():
    """C2 shape (1024 envs, 64x64 p=0.2, 128 agents): invariants over steps."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 1024, 64, 128
    grids, starts, goals = make_batch(2026, E, W, W, A)
    ext = ext_for(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * W, 7, "standard_mapf", 512)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    gt = g.bool()
    gen = torch.Generator(device="cuda").manual_seed(3)
    index = torch.arange(A, device="cuda").expand(E, A)
    # Action deltas: 0 stay, 1 x-1, 2 x+1, 3 y-1, 4 y+1.
    DX = torch.tensor([0, -1, 1, 0, 0], device="cuda")
    DY = torch.tensor([0, 0, 0, -1, 1], device="cuda")
    swaps_seen = 0
    for _ in range(16):
        before = torch.stack([sim.cur_x, sim.cur_y], -1).long()
        acts = torch.randint(0, 5, (E, A), dtype=torch.uint8, device="cuda", generator=gen)
        sim.update_actions(acts)
        sim.step_sim_only()
        after = torch.stack([sim.cur_x, sim.cur_y], -1).long()
        cells = after[..., 0] * W + after[..., 1]
        srt = cells.sort(dim=1).values
        assert not bool((srt[:, 1:] == srt[:, :-1]).any()), "shared cell"
        assert not bool(gt[torch.arange(E, device="cuda")[:, None], after[..., 0], after[..., 1]].any())
        assert bool(((after - before).abs().sum(-1) <= 1).all())
        # No swap: agent i entering the cell agent j left while j enters i's
        # old cell.  who[e, c] = agent that stood on cell c before the step.
        prev = before[..., 0] * W + before[..., 1]
        who = torch.full((E, W * W), -1, dtype=torch.long, device="cuda").scatter_(1, prev, index)
        j = who.gather(1, cells)
        moved = (cells != prev) & (j >= 0)
        swapped = moved & (cells.gather(1, j.clamp(min=0)) == prev)
        assert not bool(swapped.any()), f"swap at {swapped.nonzero()[:4].tolist()}"
        # The actions did ask for swaps: facing neighbours with opposite moves.
        want = torch.stack([before[..., 0] + DX[acts.long()], before[..., 1] + DY[acts.long()]], -1)
        wc = (want[..., 0].clamp(0, W - 1) * W + want[..., 1].clamp(0, W - 1))
        jw = who.gather(1, wc)
        swaps_seen += int(((jw >= 0) & (jw != index) & (wc != prev)
                           & (wc.gather(1, jw.clamp(min=0)) == prev)).sum())
    assert swaps_seen > 0, "no swap was requested; the invariant was not exercised"


def test_c2_full_horizon_sampled_envs_match_oracle(oracle):
    """C2 at full size over the whole 512-step horizon (and 4 steps past it):
    three sampled envs compared with the oracle after every step."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A, T = 1024, 64, 128, 512
    sample = [0, 517, 1023]
    grids, starts, goals = make_batch(2026, E, W, W, A)
    ext = ext_for(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, E * W * W, 7, "standard_mapf", T)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((E, A), dtype=torch.uint8, device="cuda"), torch.zeros(E, dtype=torch.int32, device="cuda"))
    osim = oracle.OracleSim(grids[sample], A, task_mode=1, max_episode_steps=T)
    osim.load_state(starts[sample], goals[sample])
    rng = np.random.default_rng(512)
    idx = torch.tensor(sample, device="cuda")
    rows = (idx[:, None] * A + torch.arange(A, device="cuda")).reshape(-1)
    for step in range(T + 4):
        acts = rng.integers(0, 5, size=(E, A), dtype=np.uint8)
        sim.update_actions(torch.from_numpy(acts).cuda())
        sim.step_sim_only()
        osim.step(acts[sample])
        pairs = [
            ("cur_x", sim.cur_x[idx], osim.cur_x.astype(np.int16)),
            ("cur_y", sim.cur_y[idx], osim.cur_y.astype(np.int16)),
            ("outcomes", sim.outcomes[idx], osim.outcomes),
            ("arrived", sim.arrived[idx], osim.arrived),
            ("terminated", sim.terminated[idx], osim.terminated),
            ("truncated", sim.truncated[idx], osim.truncated),
            ("step_counts", sim.step_counts[idx], osim.step_counts),
            ("rewards", sim.rewards[idx], osim.rewards),
            ("grid_ocp", sim.grid_ocp[idx], osim.grid_ocp.view(np.int32)),
            ("state_packed", sim.state_packed[rows, 1:], osim.state_packed.view(np.int16)[:, 1:]),
            ("goal_changed", sim.goal_changed_flags[idx], osim.goal_changed),
        ]
        for name, got, exp in pairs:
            got = got.cpu().numpy()
            assert np.array_equal(got, exp), f"step {step} {name} differs at {np.argwhere(got != exp)[:5].tolist()}"
        env_col = sim.state_packed[rows, 0].cpu().numpy()
        assert np.array_equal(env_col, np.repeat(np.array(sample, np.int16), A))
    assert bool((osim.truncated | osim.terminated).all())
    assert int(sim.step_counts.max()) <= T


@pytest.mark.parametrize("W,H", [(32, 32), (7, 128), (64, 64), (256, 256)])
def test_encode_map_matches_closed_form_on_gpu(W, H):
    """jl_encode_map (grid_world_cuda.cu:112-183): bit (x*H + y) & 31 of word
    (x*H + y) >> 5 is set iff grid[x, y] != 0, for any nonzero cell value."""
    ext = ext_for(W, H)
    gen = torch.Generator().manual_seed(W * 1000 + H)
    E = 3
    values = torch.randint(1, 7, (E, W, H), generator=gen, dtype=torch.int32)
    grids = torch.where(torch.rand((E, W, H), generator=gen) < 0.3, values, torch.zeros_like(values))
    grids[0] = 0
    grids[1, 0, :] = 5
    sim = ext.GridWorldSimulator(grids.cuda(), 2, 0, E * W * H, 7, "standard_mapf", 8)
    torch.cuda.synchronize()
    bits = sim.memory_tensors["grid_compressed"].cpu().numpy().view(np.uint32)
    assert bits.shape == (E, W * H // 32)
    cells = np.arange(W * H)
    got = (bits[:, cells >> 5] >> (cells & 31).astype(np.uint32)) & 1
    assert np.array_equal(got.reshape(E, W, H), (grids.numpy() != 0).astype(np.uint32))


def test_decode_to_uint8_unpacks_rows():
    """decode_to_uint8 (grid_world_cuda.cu:186-210): out[b, c, r, k] is bit k
    of the packed row agents_obs[b, c, r]."""
    ext = ext_for(32, 32)
    E, A = 3, 5
    sim = _sim(ext, num_envs=E, num_agents=A, task_mode="standard_mapf")
    obs = sim.agents_obs
    n, feats, d = obs.shape
    assert n == E * A and feats >= 2
    packed = torch.randint(0, 1 << 16, (n, feats, d), generator=torch.Generator().manual_seed(9), dtype=torch.int32)
    packed[0] = 0xFFFF
    packed[1] = 0
    obs.copy_(torch.from_numpy(packed.numpy().astype(np.uint16).view(np.int16)).cuda())
    out = sim.decode_to_uint8()
    torch.cuda.synchronize()
    assert out.shape == (n, 2, d, d) and out.dtype == torch.uint8
    rows = packed[:, :2].numpy().astype(np.uint32)
    want = (rows[..., None] >> np.arange(d, dtype=np.uint32)) & 1
    assert np.array_equal(out.cpu().numpy(), want.astype(np.uint8))


def test_step_beyond_the_full_hash_and_past_the_lds_limit(oracle):
    """On a 256x256 map the step's LDS tables at a load factor of 1/2 hold
    2,048 agents per env; 2,250 take the fuller hash (the smallest power of
    two above 2A slots) and still equal the oracle step for step, and 2,400
    are refused with the library's agent-count error, as is a token build of
    4,096 (its per-env tables would pass 160 KB of LDS too)."""
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions

    W = H = 256
    ext = profile(W, H)
    A = 2250
    print(f"[step] {W}x{H} A={A}", flush=True)
    grids, starts, goals = make_batch(2250, 1, W, H, A, density=0.1)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, W * H, 3, "standard_mapf", 64)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((1, A), dtype=torch.uint8, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda"))
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=64)
    osim.load_state(starts, goals)
    acts = random_actions(np.random.default_rng(3), 3, 1, A)
    for s in range(3):
        sim.update_actions(torch.from_numpy(acts[s]).cuda())
        sim.step_sim_only()
        osim.step(acts[s])
        compare_with_oracle(sim, osim, f"A={A} step {s}")

    A = 2400
    grids, starts, goals = make_batch(2400, 1, W, H, A, density=0.1)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    sim = ext.GridWorldSimulator(g, A, 0, W * H, 3, "standard_mapf", 64)
    sim.load_state(torch.from_numpy(starts).cuda(), torch.from_numpy(goals).cuda(),
                   torch.zeros((1, A), dtype=torch.uint8, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda"))
    sim.update_actions(torch.zeros((1, A), dtype=torch.uint8, device="cuda"))
    with pytest.raises(RuntimeError, match="too many agents per env"):
        sim.step_sim_only()
    A = 4096
    grids, starts, goals = make_batch(4096, 1, W, H, A, density=0.05)
    b = ext.MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)
    st = [torch.from_numpy(np.ascontiguousarray(v)).cuda()
          for v in (starts[..., 0], starts[..., 1], goals[..., 0], goals[..., 1])]
    with pytest.raises(RuntimeError, match="too many agents per env"):
        b.build_tokens_from_state(*st)
    torch.cuda.synchronize()
