"""CPU pins of the MAGAT / energy oracle (oracle/jl_oracle.c: jlo_energy_*,
jlo_magat_occupancy, jlo_magat_nodes, jlo_magat_edges).

Anchors:
* the reference's cell-level KATs (golden/magat_kats.json, transcribed from
  tests/expert/test_compact_state_api.py and test_cuda_kernels.py);
* an independent numpy restatement, written here from the reference's CPU
  oracle sources rather than from the CUDA kernel: POGEMA observation
  windows with the one-cell obstacle ring of add_artificial_border
  (src/pogema/grid.py:111-128, 214-222), the arctan2 goal projection of
  test_obs_consistency.py:42-70 and the normalised, clamped cost-to-go of
  CostToGoCalculator (third_party/lagat/.../cost_to_go_calculator.py:46-120);
  on maps whose distances stay below 246 the CUDA energy formula
  (E = 255 - d) is exact, so the two must agree bit for bit;
* closed forms: energy = 255 - BFS distance capped at 254, the COO edge list
  of all ordered pairs within squared radius 49 sorted by (source, target).
"""
import json
from collections import deque
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
R = 5  # OBS_RADIUS


def bfs_dist(grid, goal):
    """Exact 4-neighbour BFS distance over free cells (-1 unreachable)."""
    W, H = grid.shape
    d = np.full((W, H), -1, np.int64)
    d[goal] = 0
    q = deque([goal])
    while q:
        x, y = q.popleft()
        for nx, ny in ((x - 1, y), (x + 1, y), (x, y - 1), (x, y + 1)):
            if 0 <= nx < W and 0 <= ny < H and not grid[nx, ny] and d[nx, ny] < 0:
                d[nx, ny] = d[x, y] + 1
                q.append((nx, ny))
    return d


def pogema_style_nodes(grid, positions, goals):
    """[A, 4, 13, 13] float32 node features restated from POGEMA +
    CostToGoCalculator (independent of the CUDA kernel and of the C oracle)."""
    W, H = grid.shape
    A = len(positions)
    # padded grid: free outside, one obstacle ring at distance 1 (empty_outside)
    pad = np.zeros((W + 2 * R, H + 2 * R), np.float32)
    pad[R - 1, R - 1:H + R + 1] = 1
    pad[W + R, R - 1:H + R + 1] = 1
    pad[R - 1:W + R + 1, R - 1] = 1
    pad[R - 1:W + R + 1, H + R] = 1
    pad[R:W + R, R:H + R] = grid
    occ = np.zeros_like(pad)
    for x, y in positions:
        occ[x + R, y + R] = 1
    out = np.zeros((A, 4, 13, 13), np.float32)
    for a in range(A):
        x, y = positions[a]
        out[a, 0] = np.pad(pad[x:x + 2 * R + 1, y:y + 2 * R + 1], 1)
        out[a, 1] = np.pad(occ[x:x + 2 * R + 1, y:y + 2 * R + 1], 1)
        g = (goals[a][0] - x, goals[a][1] - y)
        if abs(g[0]) <= R and abs(g[1]) <= R:
            out[a, 2, 6 + g[0], 6 + g[1]] = 1.0
        else:
            angle = np.arctan2(g[1], g[0])
            sign = np.sign(g)
            dist = 6
            if (np.pi / 4 <= angle <= np.pi * 3 / 4) or (-np.pi * 3 / 4 <= angle <= -np.pi / 4):
                gy = int(dist * (sign[1] + 1))
                gx = int(6 + np.round(dist * g[0] / np.abs(g[1])))
            else:
                gx = int(dist * (sign[0] + 1))
                gy = int(6 + np.round(dist * g[1] / np.abs(g[0])))
            out[a, 2, gx, gy] = 1.0
        # CostToGoCalculator: invalid (off map / obstacle) -> base + 2R;
        # unreachable free cells -> grid.size
        d = bfs_dist(grid, tuple(goals[a]))
        base = d[x, y] if d[x, y] >= 0 else W * H
        ctg = np.zeros((11, 11), np.float32)
        for i in range(11):
            for j in range(11):
                cx, cy = x + i - R, y + j - R
                if not (0 <= cx < W and 0 <= cy < H) or grid[cx, cy]:
                    v = base + 2 * R
                else:
                    v = d[cx, cy] if d[cx, cy] >= 0 else W * H
                ctg[i, j] = v - base
        ctg = np.clip(ctg / np.float32(2 * R), -1.0, 1.0).astype(np.float32)
        out[a, 3] = np.pad(ctg, 1)
    return out


def random_env(rng, W, H, A, density):
    from iclr_2027_jointoom_amd.synthetic import iid_grid, place_agents

    g = iid_grid(rng, W, H, density)
    starts, goals = place_agents(rng, g, A)
    return g, starts.astype(np.int64), goals.astype(np.int64)


def state_rows(E, A, starts, goals, reset=1):
    rows = np.zeros((E * A, 8), np.uint16)
    for e in range(E):
        for a in range(A):
            r = rows[e * A + a]
            r[0], r[1] = e, a
            r[2], r[3] = starts[e][a]
            r[4], r[5] = goals[e][a]
            r[7] = reset
    return rows


def build_oracle(oracle, grids, starts, goals):
    E, W, H = grids.shape
    A = starts.shape[1]
    m = oracle.OracleMagat(grids, A)
    rows = state_rows(E, A, starts, goals)
    m.update_energy(rows, len(rows))
    rows[:, 7] = 0
    m.refresh(rows)
    m.nodes()
    m.edges()
    return m


def test_energy_closed_form_goal_cell_and_cap(oracle):
    rng = np.random.default_rng(3)
    g, _, goals = random_env(rng, 32, 32, 6, 0.25)
    for goal in goals:
        e = oracle.energy_u8(g, goal)
        d = bfs_dist(g, tuple(goal))
        want = np.where((d >= 0) & (d <= 254), 255 - np.clip(d, 0, 254), 0).astype(np.uint8)
        assert np.array_equal(e, want)
        assert e[tuple(goal)] == 255  # test_cuda_kernels.py:59-65
    # a serpentine corridor longer than 254 cells: the far end saturates to 0
    grid = np.ones((32, 32), np.uint8)
    for x in range(0, 32, 2):
        grid[x, :] = 0
        if x + 1 < 32:
            grid[x + 1, 31 if (x // 2) % 2 == 0 else 0] = 0
    d = bfs_dist(grid, (0, 0))
    assert d.max() > 300
    e = oracle.energy_u8(grid, (0, 0))
    assert e[d == 254].min() == 1 and (e[d >= 255] == 0).all()


def test_occupancy_kat(oracle):
    kat = json.loads((GOLDEN / "magat_kats.json").read_text())["occupancy"]
    grids = np.zeros((1, 128, 128), np.uint8)
    starts = np.asarray([kat["agents"]])
    goals = np.asarray([[kat["goal"]] * len(kat["agents"])])
    m = oracle.OracleMagat(grids, len(kat["agents"]))
    m.refresh(state_rows(1, len(kat["agents"]), starts, goals, reset=0))
    occ = m.grid_ocp[0]
    bit = lambda x, y: (occ[(x * 128 + y) >> 5] >> ((x * 128 + y) & 31)) & 1  # noqa: E731
    assert all(bit(x, y) for x, y in kat["set"]) and not any(bit(x, y) for x, y in kat["unset"])


def test_occupancy_skips_positions_off_the_map(oracle):
    """Rows at positions off the map (negative, at W or H, the int16
    extremes) set no bit and touch nothing outside the env's bitmap: env 0
    (every agent off the map) stays clear, env 1 (half of them off) equals
    the bitmap of its on-map rows alone, and env 2 (rows with no valid env
    id, never written) stays clear."""
    E, W, A = 3, 32, 6
    grids = np.zeros((E, W, W), np.uint8)
    starts = np.zeros((E, A, 2), np.int16)
    starts[:, :, 0] = np.arange(A)[None, :] * 3
    starts[:, :, 1] = np.arange(A)[None, :] * 5
    off = np.asarray([(-1, 0), (0, -1), (W, 0), (0, W), (-32768, 32767), (9000, -9000)], np.int16)
    far = starts.copy()
    far[0] = off
    far[1, 3:] = off[:3]
    goals = np.zeros((E, A, 2), np.int16)
    rows = state_rows(E, A, far, goals, reset=0)
    rows.reshape(E, A, 8)[2, :, 0] = 0xFFFF
    m = oracle.OracleMagat(grids, A)
    m.refresh(rows)
    on_map = state_rows(E, A, starts, goals, reset=0)
    on_map.reshape(E, A, 8)[1, 3:, 0] = 0xFFFF  # the off-map agents of env 1 left out
    ref = oracle.OracleMagat(grids, A)
    ref.refresh(on_map)
    assert not m.grid_ocp[0].any()
    assert np.array_equal(m.grid_ocp[1], ref.grid_ocp[1]) and m.grid_ocp[1].any()
    assert not m.grid_ocp[2].any()


def test_local_gather_kats(oracle):
    kat = json.loads((GOLDEN / "magat_kats.json").read_text())["local_gather"]
    A = kat["n_agents"]
    grids = np.zeros((1, 128, 128), np.uint8)
    for x, y in kat["obstacles"]:
        grids[0, x, y] = 1
    ids = np.arange(A)
    pos = np.stack([ids // 16 + 40, ids % 16 + 40], 1)
    k = ids[256:] - 256
    pos[256:] = np.stack([k // 16 + 90, k % 16 + 90], 1)
    goals = np.full((A, 2), 64)
    for a, (px, py, gx, gy) in kat["overrides"].items():
        pos[int(a)] = (px, py)
        goals[int(a)] = (gx, gy)
    m = build_oracle(oracle, grids, pos[None], goals[None])
    x = m.pyg_x.reshape(A, 4, 13, 13)
    for agent, ch, r, c, v in kat["expected_x"]:
        assert x[agent, ch, r, c] == pytest.approx(v), (agent, ch, r, c)
    assert np.array_equal(m.pyg_pos, pos.astype(np.float32))
    assert m.num_edges[0] > 0


@pytest.mark.parametrize("seed,W,A,density", [(1, 32, 24, 0.2), (2, 32, 64, 0.3), (3, 32, 12, 0.4)])
def test_nodes_match_pogema_style_restatement(oracle, seed, W, A, density):
    rng = np.random.default_rng(seed)
    g, starts, goals = random_env(rng, W, W, A, density)
    m = build_oracle(oracle, g[None], starts[None], goals[None])
    want = pogema_style_nodes(g, [tuple(p) for p in starts], [tuple(q) for q in goals])
    got = m.pyg_x.reshape(A, 4, 13, 13)
    assert np.array_equal(got, want)  # 0 ULP, float32 channels included


def test_goal_projection_covers_every_direction(oracle):
    """Goals outside the window in all directions, diagonals included."""
    g = np.zeros((64, 64), np.uint8)
    c = (32, 32)
    goals = [(32 + dx, 32 + dy) for dx in (-20, -7, -6, 0, 6, 7, 20) for dy in (-20, -7, -6, 0, 6, 7, 20)
             if max(abs(dx), abs(dy)) > R]
    goals += [(32 + 9, 32 + 9), (32 - 9, 32 + 9), (32 + 8, 32 - 24), (32 + 3, 32 + 6), (32 - 6, 32 - 3)]
    for goal in goals:
        m = build_oracle(oracle, g[None], np.asarray([[c]]), np.asarray([[goal]]))
        want = pogema_style_nodes(g, [c], [goal])
        assert np.array_equal(m.pyg_x.reshape(1, 4, 13, 13)[:, 2], want[:, 2]), goal


def test_edges_match_closed_form(oracle):
    rng = np.random.default_rng(9)
    E, W, A = 3, 32, 40
    grids = np.zeros((E, W, W), np.uint8)
    starts = np.zeros((E, A, 2), np.int64)
    goals = np.zeros((E, A, 2), np.int64)
    for e in range(E):
        grids[e], starts[e], goals[e] = random_env(rng, W, W, A, 0.2)
    m = build_oracle(oracle, grids, starts, goals)
    src, dst, attr = [], [], []
    for e in range(E):
        for a in range(A):
            for o in range(A):
                d = starts[e, a] - starts[e, o]
                if a != o and d[0] ** 2 + d[1] ** 2 <= 49:
                    src.append(e * A + a)
                    dst.append(e * A + o)
                    attr.append((d[0], d[1], abs(d[0]) + abs(d[1])))
    ei, ea = m.valid_edges()
    assert np.array_equal(ei, np.asarray([src, dst]))
    assert np.array_equal(ea, np.asarray(attr, np.float32))
    counts = np.bincount(np.asarray(src), minlength=E * A)
    assert np.array_equal(m.edge_counts, counts)
    assert np.array_equal(m.edge_prefix, np.concatenate([[0], np.cumsum(counts)]))
