"""CPU pins of the step oracle's deterministic lifelong and CostTracer modes
(oracle/jl_oracle.c: assign_candidate_goals, jlo_step).

Anchors: a known-answer case derived by hand from the rule of
assign_goals (rebuttal/online-il/tasks.py:51-65, the CPU twin of the
candidate branch of 128_agents_map_step.cu:303-330 in
rebuttal/online-rl/native/src/cuda_backend), a set-based restatement of that
function run beside the bitmap-based C oracle on seeded rollouts, and the
invariants the rule implies."""
import numpy as np
import pytest

from iclr_2027_jointoom_amd.synthetic import make_batch

LIFELONG, STANDARD, COSTTRACER = 0, 1, 2


def assign_goals_sets(positions, goals, cursors, starts, cells, reached):
    """tasks.py:51-65 as sets and tuples (raises when an agent finds no cell)."""
    reserved = {tuple(g) for g, done in zip(goals, reached) if not done}
    for i in np.flatnonzero(reached):
        begin = int(starts[i, cursors[i] % starts.shape[1]])
        for offset in range(len(cells)):
            candidate = cells[(begin + offset) % len(cells)]
            point = tuple(int(v) for v in candidate)
            if point != tuple(int(v) for v in positions[i]) and point not in reserved:
                goals[i] = candidate
                reserved.add(point)
                cursors[i] += 1
                break
        else:
            raise RuntimeError("goal assignment exhausted reachable cells")


def test_candidate_goal_kat(oracle):
    """Own cell skipped, a goal held off-goal skipped, the old goals of agents
    on their goal free again, agents served in id order."""
    grid = np.zeros((1, 32, 32), np.uint8)
    sim = oracle.OracleSim(grid, 3, task_mode=LIFELONG)
    sim.load_state(np.array([[[1, 1], [5, 5], [9, 9]]]), np.array([[[1, 2], [5, 6], [3, 3]]]))
    cells = np.array([[[1, 2], [3, 3], [7, 7], [8, 8], [1, 3]]], np.int16)
    candidates = np.array([[[0, 3], [0, 1], [4, 4]]], np.int32)
    sim.set_goal_candidates(candidates, cells, np.array([5], np.int32))
    sim.step(np.array([[4, 4, 0]], np.uint8))
    assert sim.positions()[0].tolist() == [[1, 2], [5, 6], [9, 9]]
    assert np.stack([sim.goal_x, sim.goal_y], -1)[0].tolist() == [[7, 7], [1, 2], [3, 3]]
    assert sim.goal_cursors[0].tolist() == [1, 1, 0]
    assert sim.goal_changed[0].tolist() == [1, 1, 0]
    assert sim.step_counts.tolist() == [1]
    # packed rows: the action as given and the goal-changed flag as reset flag
    rows = sim.state_packed.reshape(3, 8)
    assert rows[:, 6].tolist() == [4, 4, 0] and rows[:, 7].tolist() == [1, 1, 0]
    assert rows[:, 4:6].tolist() == [[7, 7], [1, 2], [3, 3]]
    # second step: nobody stands on a goal, so nothing changes
    sim.step(np.array([[0, 0, 0]], np.uint8))
    assert sim.goal_cursors[0].tolist() == [1, 1, 0] and sim.goal_changed[0].tolist() == [0, 0, 0]
    assert sim.step_counts.tolist() == [2]


def test_candidate_goals_match_set_restatement_on_rollouts(oracle):
    E, W, A, T = 3, 32, 24, 40
    grids, starts, goals = make_batch(17, E, W, W, A)
    rng = np.random.default_rng(3)
    cells_l = [np.argwhere(g == 0).astype(np.int16) for g in grids]
    stride = max(len(c) for c in cells_l)
    cells = np.zeros((E, stride, 2), np.int16)
    for e, c in enumerate(cells_l):
        cells[e, :len(c)] = rng.permutation(c)
    counts = np.array([len(c) for c in cells_l], np.int32)
    candidates = rng.integers(0, counts.min(), size=(E, A, 5)).astype(np.int32)
    # goals = starts for a third of the agents: they are on their goal at once
    goals = goals.copy()
    goals[:, ::3] = starts[:, ::3]
    sim = oracle.OracleSim(grids, A, task_mode=LIFELONG)
    sim.load_state(starts, goals)
    sim.set_goal_candidates(candidates, cells, counts)
    ref_goals = goals.astype(np.int64).copy()
    ref_cursors = np.zeros((E, A), np.int64)
    changed_total = 0
    for t in range(T):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        if t == 0:
            acts[:] = 0  # the agents placed on their goal stay there: all of them take new goals
        before = np.stack([sim.goal_x, sim.goal_y], -1).astype(np.int64)
        cursors_before = sim.goal_cursors.copy()
        sim.step(acts)
        pos = sim.positions().astype(np.int64)
        for e in range(E):
            reached = np.all(pos[e] == ref_goals[e], axis=1)
            assert np.array_equal(before[e], ref_goals[e])
            assign_goals_sets(pos[e], ref_goals[e], ref_cursors[e], candidates[e], cells[e, :counts[e]], reached)
        got = np.stack([sim.goal_x, sim.goal_y], -1).astype(np.int64)
        assert np.array_equal(got, ref_goals), t
        assert np.array_equal(sim.goal_cursors, ref_cursors), t
        assert np.array_equal(sim.goal_changed != 0, sim.goal_cursors != cursors_before)
        changed_total += int(sim.goal_changed.sum())
        for e in range(E):
            # goals stay distinct, and a new goal is never the agent's own cell
            assert len({tuple(g) for g in got[e]}) == A
            new = sim.goal_changed[e] != 0
            assert not np.any(np.all(got[e][new] == pos[e][new], axis=1))
        assert sim.step_counts.tolist() == [t + 1] * E
    assert changed_total >= E * len(range(0, A, 3))  # at least every agent that started on its goal


def test_costtracer_step_moves_and_counts_only(oracle):
    E, W, A = 2, 32, 16
    grids, starts, goals = make_batch(5, E, W, W, A)
    sims = {m: oracle.OracleSim(grids, A, task_mode=m) for m in (STANDARD, COSTTRACER)}
    for s in sims.values():
        s.load_state(starts, goals)
    rows_before = sims[COSTTRACER].state_packed.copy()
    rng = np.random.default_rng(8)
    for t in range(6):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        for s in sims.values():
            s.step(acts)
        a, b = sims[STANDARD], sims[COSTTRACER]
        # arrived agents of the standard mode stay; compare only while none has arrived
        if not a.arrived.any():
            assert np.array_equal(a.positions(), b.positions()), t
            assert np.array_equal(a.grid_ocp, b.grid_ocp)
        assert np.array_equal(b.rewards, (np.all(b.positions() == goals, axis=-1)).astype(np.float32))
    assert sims[COSTTRACER].step_counts.tolist() == [6, 6]
    assert np.array_equal(sims[COSTTRACER].state_packed, rows_before)  # no packed rows in this mode
    assert not sims[COSTTRACER].arrived.any() and not sims[COSTTRACER].terminated.any()


def test_set_restatement_rejects_exhaustion():
    with pytest.raises(RuntimeError, match="exhausted"):
        assign_goals_sets(np.array([[0, 0]]), np.array([[0, 0]]), np.zeros(1, np.int64),
                          np.zeros((1, 1), np.int32), np.array([[0, 0]]), np.array([True]))
