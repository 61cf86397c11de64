"""CPU pins of the oracle's generator-drawn lifelong path (oracle/jl_oracle.c:
jlo_splitmix64, jlo_xorshift64s, jlo_seed_rng, jlo_free_cells,
jlo_init_agents, assign_random_goals through jlo_step).

The reference draws from cuRAND XORWOW streams with racing threads
(128_agents_map_step.cu:265-343, grid_world_cuda.cu:405-479,
utils_cuda.h:39-61), which cannot be reproduced; this build keeps the
reference's search (start index from a draw, linear probe with wrap-around
over the env's free-cell list, goals of agents off their goal reserved) with
per-agent xorshift64* generators and agents settled in id order.  Anchors:

* SplitMix64's published outputs from state 0;
* the xorshift state update's full period 2^64 - 1 (Marsaglia 2003): its
  GF(2) matrix T satisfies T^(2^64-1) = I and T^((2^64-1)/p) != I for every
  prime p dividing 2^64 - 1, which a wrong shift amount or direction breaks;
* an independent pure-Python restatement of the generator's output;
* hand-derived known answers for the free-cell list, the placement and one
  reassignment, with generator states searched so the draws land where the
  case needs them;
* a set-based Python restatement of placement and reassignment run beside the
  bitmap-based C oracle on seeded rollouts, and the rule's invariants.
"""
import ctypes

import numpy as np

from iclr_2027_jointoom_amd.synthetic import iid_grid

M64 = (1 << 64) - 1
LIFELONG = 0


def xorshift64s(state):
    """xorshift64* (Vigna 2016): (new state, output)."""
    x = state
    x ^= x >> 12
    x ^= (x << 25) & M64
    x ^= x >> 27
    return x, (x * 0x2545F4914F6CDD1D) & M64


def draw(state, count):
    """(new state, start index) of one draw over a list of `count` entries."""
    state, out = xorshift64s(state)
    return state, (out >> 32) % count


def test_splitmix64_published_outputs(oracle):
    """SplitMix64 from state 0: 0xe220a8397b1dcdaf, 0x6e789e6aa1b965f4,
    0x06c45d188009454f, 0xf88bb8a8724c81ec; jlo_splitmix64(x) is the output
    for state x + golden, so the k-th output is jlo_splitmix64(k * golden)."""
    golden = 0x9E3779B97F4A7C15
    expected = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    got = [oracle.lib().jlo_splitmix64((k * golden) & M64) for k in range(4)]
    assert got == expected


def _c_step(oracle, v):
    st = ctypes.c_uint64(v)
    oracle.lib().jlo_xorshift64s(ctypes.byref(st))
    return st.value


def test_xorshift_state_update_has_full_period(oracle):
    """The C oracle's state update, as a GF(2)-linear map, has order exactly
    2^64 - 1 (the generator visits every nonzero state)."""
    cols = [_c_step(oracle, 1 << i) for i in range(64)]

    def apply(m, v):
        r = 0
        i = 0
        while v:
            if v & 1:
                r ^= m[i]
            v >>= 1
            i += 1
        return r

    def mul(a, b):  # a after b
        return [apply(a, c) for c in b]

    def power(m, n):
        result = [1 << i for i in range(64)]
        while n:
            if n & 1:
                result = mul(m, result)
            m = mul(m, m)
            n >>= 1
        return result

    identity = [1 << i for i in range(64)]
    # linear: the update of a sum of bits is the sum of their updates
    rng = np.random.default_rng(0)
    for v in rng.integers(1, 1 << 62, 20):
        assert _c_step(oracle, int(v)) == apply(cols, int(v))
    order = M64
    assert power(cols, order) == identity
    for p in (3, 5, 17, 257, 641, 65537, 6700417):  # 2^64 - 1 = 3 * 5 * 17 * 257 * 641 * 65537 * 6700417
        assert power(cols, order // p) != identity, p


def test_xorshift_output_matches_independent_restatement(oracle):
    rng = np.random.default_rng(1)
    for v in rng.integers(1, 1 << 63, 50, dtype=np.int64):
        c = ctypes.c_uint64(int(v))
        py = int(v)
        for _ in range(8):
            out = oracle.lib().jlo_xorshift64s(ctypes.byref(c))
            py, pout = xorshift64s(py)
            assert (c.value, out) == (py, pout)


def test_seed_rng_states(oracle):
    st = np.zeros(100, np.uint64)
    oracle.lib().jlo_seed_rng(st.ctypes.data, 100, 77)
    sm = oracle.lib().jlo_splitmix64
    assert [int(v) for v in st] == [sm(77 ^ sm(i)) or 0x9E3779B97F4A7C15 for i in range(100)]
    assert len(set(st.tolist())) == 100 and 0 not in st


def _states_with_draws(wanted, count, first=1):
    """A generator state whose successive draws over `count` entries give the
    start indices `wanted`."""
    s = first
    while True:
        st, ok = s, True
        for w in wanted:
            st, k = draw(st, count)
            if k != w:
                ok = False
                break
        if ok:
            return s
        s += 1


def test_free_cells_and_placement_kat(oracle):
    """One env, 4 x 32 map with obstacles at (0, 1) and (1, 0), real extent
    2 x 3: free cells (0,0) (0,2) (1,1) (1,2) in cell order.  Agent 0 draws
    start index 2 -> (1,1), then 2 again -> taken, probe to 3 -> (1,2);
    agent 1 draws 3 -> taken, wrap to 0 -> (0,0), then 0 -> taken, probe to
    1 -> (0,2)."""
    grid = np.zeros((1, 4, 32), np.uint8)
    grid[0, 0, 1] = grid[0, 1, 0] = 1
    sim = oracle.OracleSim(grid, 2, task_mode=LIFELONG)
    sim.seed_rng(0)
    s0, s1 = _states_with_draws([2, 2], 4), _states_with_draws([3, 0], 4)
    sim.rng_state[:] = [s0, s1]
    sim.lifelong_init(np.array([[2, 3]], np.int32))
    assert sim.env_counts.tolist() == [4] and sim.env_offsets.tolist() == [0]
    cells = [(int(c) >> 16, int(c) & 0xFFFF) for c in sim.free_cells[:4]]
    assert cells == [(0, 0), (0, 2), (1, 1), (1, 2)]
    assert sim.positions()[0].tolist() == [[1, 1], [0, 0]]
    assert np.stack([sim.goal_x, sim.goal_y], -1)[0].tolist() == [[1, 2], [0, 2]]
    assert [int(v) for v in sim.rng_state] == [draw(draw(s, 4)[0], 4)[0] for s in (s0, s1)]
    # an env with no free cell inside its extent: offset -1, no draws
    empty = oracle.OracleSim(np.ones((1, 4, 32), np.uint8), 1, task_mode=LIFELONG)
    empty.seed_rng(3)
    before = empty.rng_state.copy()
    empty.lifelong_init()
    assert empty.env_counts.tolist() == [0] and empty.env_offsets.tolist() == [-1]
    assert np.array_equal(empty.rng_state, before)
    assert empty.positions()[0].tolist() == [[-1, -1]]  # 0xFFFF: no cell


def test_reassignment_kat_on_an_open_map(oracle):
    """One env, 1 x 32 map, extent 1 x 4: cells (0,0) (0,1) (0,2) (0,3).
    Agents start at (0,0) and (0,3) with goals (0,1) and (0,3): agent 1 is on
    its goal.  Step with agent 0 moving right onto (0,1) (its goal) and agent
    1 waiting: both draw, in id order.  Agent 0 draws 3 -> (0,3): not
    reserved (agent 1 is on its goal), taken.  Agent 1 draws 3 -> taken by
    agent 0, probe wraps to 0 -> (0,0), taken.  Goals (0,3) and (0,0), both
    flagged; the generators advanced once each.  Next step both wait off
    their goals: nothing is drawn."""
    grid = np.zeros((1, 1, 32), np.uint8)
    sim = oracle.OracleSim(grid, 2, task_mode=LIFELONG)
    sim.seed_rng(0)
    sim.lifelong_init(np.array([[1, 4]], np.int32))
    s0, s1 = _states_with_draws([3], 4), _states_with_draws([3], 4, first=10 ** 6)
    sim.rng_state[:] = [s0, s1]
    sim.load_state(np.array([[[0, 0], [0, 3]]]), np.array([[[0, 1], [0, 3]]]))
    sim.step(np.array([[4, 0]], np.uint8))
    assert sim.positions()[0].tolist() == [[0, 1], [0, 3]]
    assert np.stack([sim.goal_x, sim.goal_y], -1)[0].tolist() == [[0, 3], [0, 0]]
    assert sim.goal_changed[0].tolist() == [1, 1]
    assert [int(v) for v in sim.rng_state] == [draw(s0, 4)[0], draw(s1, 4)[0]]
    rows = sim.state_packed.reshape(2, 8)
    assert rows[:, 4:6].tolist() == [[0, 3], [0, 0]] and rows[:, 7].tolist() == [1, 1]
    assert rows[:, 6].tolist() == [4, 0]
    assert sim.step_counts.tolist() == [0]  # the generator-drawn branch counts no step (:265-361)
    before = sim.rng_state.copy()
    sim.step(np.array([[0, 0]], np.uint8))
    assert sim.goal_changed[0].tolist() == [0, 0]
    assert np.array_equal(sim.rng_state, before)


def place_sets(free, states, A):
    """init_agents as Python sets: per agent a start, then a goal."""
    taken, starts, goals = set(), [], []
    for a in range(A):
        picked = []
        for _ in range(2):
            states[a], k = draw(states[a], len(free))
            for off in range(len(free)):
                j = (k + off) % len(free)
                if j not in taken:
                    taken.add(j)
                    picked.append(free[j])
                    break
        starts.append(picked[0])
        goals.append(picked[1])
    return starts, goals


def reassign_sets(free, states, pos, goals):
    """The random reassignment as Python sets; returns the changed flags."""
    on_goal = [tuple(p) == tuple(g) for p, g in zip(pos, goals)]
    reserved = {tuple(g) for g, done in zip(goals, on_goal) if not done}
    changed = [0] * len(goals)
    for i, done in enumerate(on_goal):
        if not done:
            continue
        states[i], k = draw(states[i], len(free))
        for off in range(len(free)):
            c = free[(k + off) % len(free)]
            if c not in reserved:
                reserved.add(c)
                goals[i] = c
                changed[i] = 1
                break
    return changed


def test_random_goals_match_set_restatement_on_rollouts(oracle):
    E, W, H, A, T = 3, 40, 32, 24, 60
    rng = np.random.default_rng(21)
    grids = np.stack([iid_grid(rng, W, H, 0.25) for _ in range(E)])
    extents = np.array([[40, 32], [30, 20], [17, 29]], np.int32)
    sim = oracle.OracleSim(grids, A, task_mode=LIFELONG)
    sim.seed_rng(1234)
    states = [[int(v) for v in sim.rng_state[e * A:(e + 1) * A]] for e in range(E)]
    sim.lifelong_init(extents)
    free = [[(x, y) for x in range(min(W, rw)) for y in range(min(H, rh)) if grids[e, x, y] == 0]
            for e, (rw, rh) in enumerate(extents)]
    goals = []
    for e in range(E):
        assert sim.env_counts[e] == len(free[e])
        listed = [(int(c) >> 16, int(c) & 0xFFFF) for c in sim.free_cells[e * W * H:e * W * H + len(free[e])]]
        assert listed == free[e]
        s, g = place_sets(free[e], states[e], A)
        assert [tuple(p) for p in sim.positions()[e].tolist()] == s
        goals.append(g)
    changed_total = 0
    for t in range(T):
        acts = rng.integers(0, 5, size=(E, A)).astype(np.uint8)
        sim.step(acts)
        pos = [[tuple(p) for p in sim.positions()[e].tolist()] for e in range(E)]
        for e in range(E):
            flags = reassign_sets(free[e], states[e], pos[e], goals[e])
            got = [tuple(g) for g in np.stack([sim.goal_x[e], sim.goal_y[e]], -1).tolist()]
            assert got == goals[e], (t, e)
            assert sim.goal_changed[e].tolist() == flags, (t, e)
            assert [int(v) for v in sim.rng_state[e * A:(e + 1) * A]] == states[e], (t, e)
            # invariants: goals distinct, on free cells inside the real extent
            assert len(set(got)) == A
            assert all(grids[e][g] == 0 and g[0] < extents[e][0] and g[1] < extents[e][1] for g in got)
            changed_total += sum(flags)
    assert changed_total > 0
    assert sim.step_counts.tolist() == [0] * E
