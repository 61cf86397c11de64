"""CPU pins of the step oracle (oracle/jl_oracle.c: jlo_step, jlo_resolve_env).

Anchors: the reference's directed KATs (golden/directed_fixtures.json), its
stateful standard-MAPF KATs (test_stateful_standard_mapf.py), its 512-agent
chain, and an independent brute-force Jacobi scan written here from the
round rule of 128_agents_map_step.cu:91-169.
"""
import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
MOVES = np.asarray([[0, 0], [-1, 0], [1, 0], [0, -1], [0, 1]])
FIELDS = {1: "wall_rejections", 2: "vertex_rejections", 3: "edge_swap_rejections", 4: "chain_rejections"}


def brute_force(grid, current, arrived, actions):
    """Independent O(A^2)-per-round Jacobi scan (positions, categories)."""
    current = np.asarray(current, dtype=np.int64)
    arrived = np.asarray(arrived, dtype=bool)
    actions = np.asarray(actions)
    eff = np.where(arrived | (actions > 4), 0, actions)
    raw = current + MOVES[eff]
    W, H = grid.shape
    bad = (raw[:, 0] < 0) | (raw[:, 0] >= W) | (raw[:, 1] < 0) | (raw[:, 1] >= H)
    safe = np.clip(raw, [0, 0], [W - 1, H - 1])
    bad |= grid[safe[:, 0], safe[:, 1]] != 0
    prop = np.where(bad[:, None], current, raw)
    cat = np.zeros(len(current), np.uint8)
    cat[(~arrived) & (eff != 0) & bad] = 1
    for _ in range(len(current)):
        nxt = prop.copy()
        changed = False
        for i in range(len(current)):
            if (prop[i] == current[i]).all():
                continue
            c = 0
            for k in range(len(current)):
                if k == i:
                    continue
                if (prop[i] == current[k]).all() and (prop[k] == current[i]).all():
                    c = 3
                elif i > k and (prop[i] == prop[k]).all():
                    c = 2
                elif (prop[i] == current[k]).all() and (prop[k] == current[k]).all():
                    c = 4
                if c:
                    break
            if c:
                nxt[i] = current[i]
                if not cat[i]:
                    cat[i] = c
                changed = True
        prop = nxt
        if not changed:
            break
    return prop, cat


def _fixture_cases():
    return json.loads((GOLDEN / "directed_fixtures.json").read_text())


@pytest.mark.parametrize("name", list(_fixture_cases()["cases"]))
@pytest.mark.parametrize("naive", [False, True])
def test_directed_fixtures(oracle, name, naive):
    data = _fixture_cases()
    case = data["cases"][name]
    size = data["map_size"]
    grid = np.zeros((1, size, size), np.uint8)
    for x, y in case.get("walls", []):
        grid[0, x, y] = 1
    A = len(case["actions"])
    sim = oracle.OracleSim(grid, A, task_mode=1, max_episode_steps=1)
    arrived = np.asarray([case.get("arrived", [False] * A)], np.uint8)
    sim.load_state(np.asarray([case["positions"]]), np.asarray([case["goals"]]), arrived, [0])
    sim.step(np.asarray([case["actions"]], np.uint8), naive=naive)
    assert sim.positions()[0].tolist() == case["expected"]
    assert sim.terminated.astype(bool).tolist() == case.get("terminated", [False])
    assert sim.truncated.astype(bool).tolist() == case.get("truncated", [True])
    assert sim.step_counts.tolist() == [1]
    counts = {f: int((sim.outcomes == c).sum()) for c, f in FIELDS.items()}
    for field in FIELDS.values():
        assert counts[field] == case["collision"].get(field, 0), field


def test_resolvers_match_brute_force_on_seeded_cases(oracle):
    rng = np.random.default_rng(9917)
    for trial in range(200):
        A = int(rng.integers(2, 24))
        side = 12
        flat = rng.choice(side * side, size=A, replace=False)
        cur = np.stack((flat // side, flat % side), -1)
        grid = (rng.random((side, side)) < 0.12).astype(np.uint8)
        grid[cur[:, 0], cur[:, 1]] = 0
        arrived = rng.random(A) < 0.15
        actions = rng.integers(0, 6, size=A).astype(np.uint8)  # 5 = out of range -> wait
        exp_pos, exp_cat = brute_force(grid, cur, arrived, actions)
        # oracle maps must have W*H % 32 == 0: embed 12x12 in 12x32 behind walls
        big = np.ones((side, 32), np.uint8)
        big[:, :side] = grid
        for naive in (False, True):
            pos, cat = oracle.resolve_env(big, cur, arrived.astype(np.uint8), actions, naive=naive)
            assert np.array_equal(pos, exp_pos), (trial, naive)
            assert np.array_equal(cat, exp_cat), (trial, naive)


def test_event_resolver_512_agent_chain(oracle):
    A = 512
    cur = np.stack((np.zeros(A, np.int32), np.arange(A, dtype=np.int32)), -1)
    grid = np.zeros((1, 544), np.uint8)
    actions = np.full(A, 4, np.uint8)
    actions[-1] = 0
    pos, cat = oracle.resolve_env(grid, cur, None, actions)
    assert np.array_equal(pos, cur)
    assert np.all(cat[:-1] == 4) and cat[-1] == 0


def test_random_rollout_invariants(oracle):
    """No shared cells, no swaps, moves are unit steps in the action direction."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(3, 4, 32, 32, 64)
    sim = oracle.OracleSim(grids, 64, task_mode=1, max_episode_steps=128)
    sim.load_state(starts, goals)
    rng = np.random.default_rng(5)
    for _ in range(64):
        before = sim.positions().astype(np.int64)
        acts = rng.integers(0, 5, size=(4, 64)).astype(np.uint8)
        was_done = (sim.terminated | sim.truncated).astype(bool)
        sim.step(acts)
        after = sim.positions().astype(np.int64)
        for e in range(4):
            if was_done[e]:
                assert np.array_equal(after[e], before[e])
                continue
            cells = after[e, :, 0] * 32 + after[e, :, 1]
            assert len(np.unique(cells)) == 64
            moved = np.any(after[e] != before[e], axis=1)
            assert np.array_equal(after[e][moved] - before[e][moved], MOVES[acts[e][moved]])
            assert np.all(sim.outcomes[e][moved] == 0)
            for i in np.flatnonzero(moved):
                j = np.flatnonzero((after[e] == before[e][i]).all(1) & (before[e] == after[e][i]).all(1))
                assert len(j) == 0, "swap"
            assert np.all(grids[e][after[e, :, 0], after[e, :, 1]] == 0)


def _sim(oracle, A=1, E=1, horizon=256):
    return oracle.OracleSim(np.zeros((E, 128, 128), np.uint8), A, task_mode=1, max_episode_steps=horizon)


def test_load_state_layout_kat(oracle):
    """test_stateful_standard_mapf.py:124-161."""
    sim = _sim(oracle, A=2, E=2)
    positions = [[[2, 3], [4, 35]], [[7, 8], [9, 10]]]
    goals = [[[2, 3], [6, 7]], [[11, 12], [13, 14]]]
    sim.load_state(positions, goals, [[1, 0], [0, 0]], [3, 4])
    assert sim.cur_x.tolist() == [[2, 4], [7, 9]]
    assert sim.cur_y.tolist() == [[3, 35], [8, 10]]
    assert sim.step_counts.tolist() == [3, 4]
    assert not sim.terminated.any() and not sim.truncated.any()
    assert sim.goal_changed.all()
    expected = np.zeros((2, 512), np.uint32)
    for e, env in enumerate(positions):
        for x, y in env:
            expected[e, x * 4 + (y >> 5)] |= np.uint32(1 << (y & 31))
    assert np.array_equal(sim.grid_ocp, expected)
    assert sim.state_packed.tolist() == [
        [0, 0, 2, 3, 2, 3, 0, 1],
        [0, 1, 4, 35, 6, 7, 0, 1],
        [1, 0, 7, 8, 11, 12, 0, 1],
        [1, 1, 9, 10, 13, 14, 0, 1],
    ]


def test_standard_mode_kats(oracle):
    """test_stateful_standard_mapf.py:451-514."""
    # arrived agent stays and occupies its goal
    sim = _sim(oracle, A=2)
    sim.load_state([[[10, 10], [11, 10]]], [[[10, 10], [20, 20]]], [[1, 0]])
    sim.step([[2, 1]])
    assert sim.cur_x.tolist() == [[10, 11]] and sim.cur_y.tolist() == [[10, 10]]
    assert int(sim.grid_ocp[0, 10 * 4]) & (1 << 10)
    assert sim.arrived.tolist() == [[1, 0]]
    assert sim.state_packed[:, 6].tolist() == [0, 1]
    # final arrival terminates
    sim = _sim(oracle)
    sim.load_state([[[10, 10]]], [[[11, 10]]])
    sim.step([[2]])
    assert sim.cur_x.tolist() == [[11]] and sim.arrived.tolist() == [[1]]
    assert sim.terminated.tolist() == [1] and sim.truncated.tolist() == [0]
    # horizon truncates; termination at the horizon wins
    sim = _sim(oracle, horizon=3)
    sim.load_state([[[10, 10]]], [[[20, 20]]], None, [2])
    sim.step([[0]])
    assert sim.step_counts.tolist() == [3] and sim.truncated.tolist() == [1]
    sim = _sim(oracle, horizon=3)
    sim.load_state([[[10, 10]]], [[[11, 10]]], None, [2])
    sim.step([[2]])
    assert sim.terminated.tolist() == [1] and sim.truncated.tolist() == [0]
    # done env no longer advances
    before = (sim.cur_x.copy(), sim.step_counts.copy(), sim.state_packed.copy(), sim.grid_ocp.copy())
    sim.step([[2]])
    after = (sim.cur_x, sim.step_counts, sim.state_packed, sim.grid_ocp)
    assert all(np.array_equal(a, b) for a, b in zip(before, after))


@pytest.mark.parametrize("W,H", [(32, 32), (64, 64), (7, 128), (256, 256)])
def test_encode_map_closed_form(oracle, W, H):
    """grid_world_cuda.h:17-23: word = cell >> 5, bit = cell & 31, cell = x*H + y."""
    rng = np.random.default_rng(W * 1000 + H)
    grids = (rng.random((2, W, H)) < 0.3).astype(np.int32) * rng.integers(1, 7, size=(2, W, H))
    bits = oracle.encode(grids)
    assert bits.shape == (2, W * H // 32)
    cells = np.arange(W * H)
    got = (bits[:, cells >> 5] >> (cells & 31).astype(np.uint32)) & 1
    assert np.array_equal(got.reshape(2, W, H), (grids != 0).astype(np.uint32))
