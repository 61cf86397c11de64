"""CPU pins of the BFS and MAPF-GPT oracle (oracle/jl_oracle.c).

Anchors: the reference tokenizer KATs (golden/mapfgpt_kats.json), the uint16
corridor KAT, closed forms on obstacle-free maps (BFS distance = Manhattan
distance, so every cost, coordinate, history and greedy token has a closed
form), and an independent Bellman-Ford relaxation for the BFS on random maps.
"""
import json
from pathlib import Path

import numpy as np
import pytest

KATS = json.loads((Path(__file__).resolve().parent / "golden" / "mapfgpt_kats.json").read_text())


def embed(grid: np.ndarray, W: int | None = None, H: int = 32) -> np.ndarray:
    """Pad a small map with obstacles to a profile shape (same tokens: an
    obstacle and the map edge are both unreachable cost 0xFFFF)."""
    w, h = grid.shape
    W = W or w
    out = np.ones((W, H), np.uint8)
    out[:w, :h] = grid
    return out


def relax_distances(grid: np.ndarray, goal) -> np.ndarray:
    """Bellman-Ford style fixed point: d = min(d, d_neighbour + 1) on free cells."""
    W, H = grid.shape
    INF = 1 << 30
    d = np.full((W + 2, H + 2), INF, np.int64)
    free = np.zeros((W + 2, H + 2), bool)
    free[1:-1, 1:-1] = grid == 0
    if grid[goal] != 0:
        return np.full((W, H), 65535, np.uint16)
    d[goal[0] + 1, goal[1] + 1] = 0
    while True:
        nb = np.minimum.reduce([d[:-2, 1:-1], d[2:, 1:-1], d[1:-1, :-2], d[1:-1, 2:]]) + 1
        inner = np.where(free[1:-1, 1:-1], np.minimum(d[1:-1, 1:-1], nb), INF)
        if np.array_equal(inner, d[1:-1, 1:-1]):
            break
        d[1:-1, 1:-1] = inner
    out = d[1:-1, 1:-1]
    return np.where(out >= INF, 65535, out).astype(np.uint16)


def test_bfs_corridor_distance_256(oracle):
    k = KATS["corridor_distance"]
    n = k["map_size"]
    grid = np.ones((n, n), np.uint8)
    for r in k["free_rows"]:
        grid[r, :] = 0
    for x, y in k["free_cells"]:
        grid[x, y] = 0
    field, bad, overflow = oracle.bfs_u16(grid, k["goal"])
    assert bad == 0 and overflow == 0
    for key, value in k["expect"].items():
        x, y = map(int, key.split(","))
        assert int(field[x, y]) == value


def test_bfs_closed_form_on_empty_map(oracle):
    W, H = 40, 64
    grid = np.zeros((W, H), np.uint8)
    for goal in [(0, 0), (17, 33), (39, 63)]:
        field, bad, _ = oracle.bfs_u16(grid, goal)
        xs, ys = np.meshgrid(np.arange(W), np.arange(H), indexing="ij")
        assert bad == 0
        assert np.array_equal(field, (np.abs(xs - goal[0]) + np.abs(ys - goal[1])).astype(np.uint16))


def test_bfs_matches_relaxation_on_random_maps(oracle):
    rng = np.random.default_rng(11)
    for _ in range(40):
        grid = (rng.random((24, 32)) < rng.uniform(0.1, 0.45)).astype(np.uint8)
        goal = tuple(int(v) for v in rng.integers(0, [24, 32]))
        field, bad, _ = oracle.bfs_u16(grid, goal)
        assert bad == int(grid[goal] != 0)
        assert np.array_equal(field, relax_distances(grid, goal))


def test_bfs_rejects_obstacle_and_off_map_goal(oracle):
    grid = np.zeros((32, 32), np.uint8)
    grid[3, 4] = 1
    for goal in [(3, 4), (32, 0), (0, 40)]:
        field, bad, _ = oracle.bfs_u16(grid, goal)
        assert bad == 1 and np.all(field == 65535)


def test_energy_closed_form_and_cap(oracle):
    grid = np.zeros((64, 64), np.uint8)
    e = oracle.energy_u8(grid, (10, 20))
    xs, ys = np.meshgrid(np.arange(64), np.arange(64), indexing="ij")
    d = np.abs(xs - 10) + np.abs(ys - 20)
    assert int(e[10, 20]) == 255
    assert np.array_equal(e, np.where(d <= 254, 255 - d, 0).astype(np.uint8))
    # snake corridor: distances beyond 254 read 0, exactly like unreachable
    grid = np.ones((32, 32), np.uint8)
    grid[::2, :] = 0
    for r in range(1, 32, 2):
        grid[r, 31 if (r // 2) % 2 == 0 else 0] = 0
    dist = relax_distances(grid, (0, 0)).astype(np.int64)
    e = oracle.energy_u8(grid, (0, 0))
    exp = np.where((dist <= 254) & (grid == 0), 255 - dist, 0)
    exp[0, 0] = 255
    assert dist.max() > 300 and np.array_equal(e, exp.astype(np.uint8))
    # goal on an obstacle still seeds the BFS (energy_map.cu:154-166)
    grid = np.zeros((32, 32), np.uint8)
    grid[5, 5] = 1
    e = oracle.energy_u8(grid, (5, 5))
    assert int(e[5, 5]) == 255 and int(e[5, 6]) == 254


def _tokenize(oracle, grid, rows, A):
    b = oracle.OracleMapfGPT(grid[None], A)
    b.build_rows(np.asarray(rows, np.uint16))
    return b


def test_tokenizer_vocabulary_and_neighbor_histories(oracle):
    k = KATS["vocabulary_and_histories"]
    grid = embed(np.zeros(k["grid_shape"], np.uint8))
    b = _tokenize(oracle, grid, k["rows"], 3)
    t = b.tokens
    assert b.labels.tolist() == k["labels"]
    assert np.all((t >= 0) & (t <= 66))
    for start, expected in k["ego0_history_slots"].items():
        s = int(start)
        assert t[0, s + 4 : s + 9].tolist() == expected
    assert np.all(t[0, k["ego0_padding_from"] :] == 66)
    assert b.diagnostics.tolist() == [0, 0, 0, 0]


def test_tokenizer_sentinels(oracle):
    k = KATS["sentinels"]
    g = np.zeros(k["grid_shape"], np.uint8)
    g[k["wall_rows_from"] :, k["wall_column"]] = 1
    b = _tokenize(oracle, embed(g, W=32, H=64), k["rows"], 2)
    t = b.tokens
    for v in k["ego0_cost_contains"]:
        assert v in t[0, :121]
    for v in k["ego1_cost_contains"]:
        assert v in t[1, :121]
    assert t[0, 123] == k["ego0_token_123"] and t[0, 124] == k["ego0_token_124"]


def test_tokenizer_top13_by_manhattan_then_id(oracle):
    positions = [(10, 10)] + [(10 + dx, 10 + dy) for dx in range(-2, 3) for dy in range(-2, 3) if (dx, dy) != (0, 0)]
    positions = positions[:16]
    rows = np.zeros((16, 13), np.uint16)
    rows[:, 1] = np.arange(16)
    rows[:, 2:4] = positions
    rows[:, 4:6] = positions
    rows[:, 7] = 1
    rows[:, 8:13] = 5
    b = _tokenize(oracle, embed(np.zeros((20, 20), np.uint8)), rows, 16)
    records = b.tokens[0, 121:251].reshape(13, 10)
    got = [tuple((r[:2] - 20).tolist()) for r in records]
    ids = sorted(range(16), key=lambda i: (abs(positions[i][0] - 10) + abs(positions[i][1] - 10), i))[:13]
    assert got == [(positions[i][0] - 10, positions[i][1] - 10) for i in ids]


def closed_form_tokens(pos, goals, hist, W, H):
    """Tokens on an obstacle-free WxH map, from Manhattan distances only."""
    A = len(pos)
    out = np.full((A, 256), 66, np.int64)
    clip = lambda v: max(-20, min(20, v)) + 20  # noqa: E731
    for e in range(A):
        ex, ey = pos[e]
        c = abs(ex - goals[e][0]) + abs(ey - goals[e][1])
        t = 0
        for dx in range(-5, 6):
            for dy in range(-5, 6):
                x, y = ex + dx, ey + dy
                if 0 <= x < W and 0 <= y < H:
                    v = abs(x - goals[e][0]) + abs(y - goals[e][1]) - c
                    out[e, t] = 43 if v > 20 else (42 if v < -20 else v + 20)
                else:
                    out[e, t] = 41
                t += 1
        vis = [j for j in range(A) if abs(pos[j][0] - ex) <= 5 and abs(pos[j][1] - ey) <= 5]
        vis.sort(key=lambda j: (abs(pos[j][0] - ex) + abs(pos[j][1] - ey), j))
        for s, j in enumerate(vis[:13]):
            base = 121 + 10 * s
            out[e, base : base + 4] = [clip(pos[j][0] - ex), clip(pos[j][1] - ey),
                                       clip(goals[j][0] - ex), clip(goals[j][1] - ey)]
            out[e, base + 4 : base + 9] = [44 if a == 5 else 45 + a for a in hist[j]]
            mask = 0
            for d, (mx, my) in enumerate(((-1, 0), (1, 0), (0, -1), (0, 1))):
                x, y = pos[j][0] + mx, pos[j][1] + my
                if 0 <= x < W and 0 <= y < H:
                    if abs(x - goals[j][0]) + abs(y - goals[j][1]) < abs(pos[j][0] - goals[j][0]) + abs(pos[j][1] - goals[j][1]):
                        mask |= 1 << (3 - d)
            out[e, base + 9] = 50 + mask
    return out


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_tokens_closed_form_on_empty_map(oracle, seed):
    rng = np.random.default_rng(seed)
    W, H, A = 24, 32, 48
    cells = rng.choice(W * H, size=A, replace=False)
    pos = [(int(c) // H, int(c) % H) for c in cells]
    gcells = rng.choice(W * H, size=A, replace=False)
    goals = [(int(c) // H, int(c) % H) for c in gcells]
    hist = rng.integers(0, 6, size=(A, 5))
    rows = np.zeros((A, 13), np.uint16)
    rows[:, 1] = np.arange(A)
    rows[:, 2:4] = pos
    rows[:, 4:6] = goals
    rows[:, 6] = rng.integers(0, 5, size=A)
    rows[:, 8:13] = hist
    b = _tokenize(oracle, np.zeros((W, H), np.uint8), rows, A)
    assert np.array_equal(b.tokens, closed_form_tokens(pos, goals, hist, W, H))
    assert b.active_mask.tolist() == [int(p != g) for p, g in zip(pos, goals)]
    assert b.labels.tolist() == rows[:, 6].tolist()


def test_history_roll_and_active_mask(oracle):
    k = KATS["history_roll"]
    b = oracle.OracleMapfGPT(np.zeros((1, 32, 32), np.uint8), 3)
    cur = np.asarray(k["cur"]).T[:, None, :]
    goal = np.asarray(k["goal"]).T[:, None, :]
    b.build_state(cur[0], cur[1], goal[0], goal[1])
    assert b.active_mask.astype(bool).tolist() == k["active"]
    b.append(np.asarray([k["actions"]], np.uint8))
    assert b.histories.tolist() == k["histories_after"]


def test_goal_cache_refresh_and_diagnostics(oracle):
    b = oracle.OracleMapfGPT(np.zeros((1, 32, 32), np.uint8), 1)
    row_a = np.asarray([[0, 0, 10, 10, 10, 20, 0, 0, 5, 5, 5, 5, 5]], np.uint16)
    row_b = row_a.copy()
    row_b[0, 4:6] = [30, 30]
    b.build_rows(row_a)
    cost_a = b.cost_to_go.copy()
    b.build_rows(row_b)
    assert b.cost_to_go[0, 0, 30, 30] == 0 and not np.array_equal(cost_a, b.cost_to_go)
    b.build_rows(row_a)
    assert np.array_equal(cost_a, b.cost_to_go)
    # a row naming the wrong agent is rejected and counted
    bad = row_a.copy()
    bad[0, 1] = 3
    b.build_rows(bad)
    assert b.diagnostics.tolist() == [0, 1, 0, 0]
    # an agent off the map: diagnostics[3], tokens stay padding
    off = row_a.copy()
    off[0, 2] = 32
    b.build_rows(off)
    assert b.diagnostics[3] > 0 and np.all(b.tokens == 66)
