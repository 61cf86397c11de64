"""Python restatement of the reference's cached CPU input builder.

TEST INFRASTRUCTURE / CPU BASELINE ONLY (bench.py's cpu_baseline leg and
tests).  It keeps the algorithm and granularity of the reference CPU path so
that its timing is a fair baseline:

* ``CachedTokenBuilder.build`` follows CachedHostBuilder.build for the
  mapf_gpt backend (src/mapf_cuda/training/host_inputs.py:99-112): a per-env
  goal cache, a ``collections.deque`` BFS for every changed goal
  (expert/mapf_gpt_schema.py:172-193) and a per-ego Python tokenizer loop
  (tokenize_stage_reference, mapf_gpt_schema.py:234-320);
* ``resolve_step`` follows the event-indexed resolver _resolve_proposals
  (expert/transition_adapters.py:361-455) plus the standard-MAPF bookkeeping
  of _predict_backend_step (:663-707);
* ``run_stage_worker`` runs one whole stage (all envs of the sample) per
  worker process, as HostPrefetch does (host_inputs.py:181-232);
* ``run_magat_worker`` does the same for the stateful MAGAT step with the C
  restatement of the step, occupancy, node and edge passes.
"""
from __future__ import annotations

from collections import deque

import numpy as np

MOVES = ((0, 0), (-1, 0), (1, 0), (0, -1), (0, 1))
UNREACHED = 65535


def bfs_cost(grid: np.ndarray, goal) -> np.ndarray:
    W, H = grid.shape
    dist = np.full((W, H), UNREACHED, dtype=np.uint16)
    gx, gy = int(goal[0]), int(goal[1])
    if not (0 <= gx < W and 0 <= gy < H) or grid[gx, gy]:
        return dist
    dist[gx, gy] = 0
    queue = deque([(gx, gy)])
    while queue:
        x, y = queue.popleft()
        nd = int(dist[x, y]) + 1
        for dx, dy in MOVES[1:]:
            nx, ny = x + dx, y + dy
            if 0 <= nx < W and 0 <= ny < H and not grid[nx, ny] and dist[nx, ny] == UNREACHED:
                dist[nx, ny] = nd
                queue.append((nx, ny))
    return dist


def _cost_tok(v, c):
    if v == UNREACHED:
        return 41
    d = v - c
    return 43 if d > 20 else (42 if d < -20 else d + 20)


def _clip(v):
    return max(-20, min(20, v)) + 20


def tokenize_env(grid, positions, goals, histories, costs, out):
    """Tokens of one env's agents into ``out`` (int32 [A, 256], pre-filled 66)."""
    W, H = grid.shape
    A = len(positions)
    for e in range(A):
        ex, ey = positions[e]
        cmap = costs[e]
        center = int(cmap[ex, ey]) if (0 <= ex < W and 0 <= ey < H) else UNREACHED
        t = 0
        row = out[e]
        for dx in range(-5, 6):
            x = ex + dx
            for dy in range(-5, 6):
                y = ey + dy
                v = int(cmap[x, y]) if (0 <= x < W and 0 <= y < H) else UNREACHED
                row[t] = _cost_tok(v, center)
                t += 1
        visible = [j for j in range(A) if abs(positions[j][0] - ex) <= 5 and abs(positions[j][1] - ey) <= 5]
        visible.sort(key=lambda j: (abs(positions[j][0] - ex) + abs(positions[j][1] - ey), j))
        for s, j in enumerate(visible[:13]):
            b = 121 + 10 * s
            px, py = positions[j]
            row[b] = _clip(px - ex)
            row[b + 1] = _clip(py - ey)
            row[b + 2] = _clip(goals[j][0] - ex)
            row[b + 3] = _clip(goals[j][1] - ey)
            for k in range(5):
                a = int(histories[j][k])
                row[b + 4 + k] = 44 if a == 5 else 45 + a
            cj = costs[j]
            cur = int(cj[px, py])
            mask = 0
            for d, (mx, my) in enumerate(MOVES[1:]):
                x, y = px + mx, py + my
                nb = int(cj[x, y]) if (0 <= x < W and 0 <= y < H) else UNREACHED
                if nb != UNREACHED and cur > nb:
                    mask |= 1 << (3 - d)
            row[b + 9] = 50 + mask


class CachedTokenBuilder:
    """Per-env goal cache + deque BFS + per-ego tokenizer (mapf_gpt backend)."""

    def __init__(self, grids: np.ndarray, n_agents: int, bfs=bfs_cost):
        self.grids = np.asarray(grids, dtype=np.uint8)
        self.A = int(n_agents)
        self.goals = [None] * len(self.grids)
        self.costs = [[None] * self.A for _ in range(len(self.grids))]
        self.rebuilds = 0
        self.bfs = bfs

    def build(self, rows: np.ndarray):
        """rows: uint16 [E*A, 13] env-major.  Returns (tokens, labels, active)."""
        E, A = len(self.grids), self.A
        blocks = rows.reshape(E, A, 13)
        tokens = np.full((E * A, 256), 66, dtype=np.int32)
        for e in range(E):
            blk = blocks[e]
            goals = blk[:, 4:6].astype(np.int64)
            if self.goals[e] is None:
                changed = np.ones(A, bool)
            else:
                changed = np.any(self.goals[e] != goals, axis=1)
            changed |= blk[:, 7] != 0
            for a in np.flatnonzero(changed):
                self.costs[e][a] = self.bfs(self.grids[e], goals[a])
                self.rebuilds += 1
            self.goals[e] = goals
            positions = [(int(x), int(y)) for x, y in blk[:, 2:4]]
            goal_list = [(int(x), int(y)) for x, y in goals]
            tokenize_env(self.grids[e], positions, goal_list, blk[:, 8:13], self.costs[e],
                         tokens[e * A:(e + 1) * A])
        labels = rows[:, 6].astype(np.int64)
        active = np.any(rows[:, 2:4] != rows[:, 4:6], axis=1)
        return tokens, labels, active


def resolve_step(grid, positions, goals, arrived, actions):
    """One env, one standard-MAPF step: (new positions, new arrived)."""
    W, H = grid.shape
    A = len(positions)
    cur = [(int(p[0]), int(p[1])) for p in positions]
    prop = []
    for i in range(A):
        act = int(actions[i])
        if arrived[i] or act > 4:
            act = 0
        x, y = cur[i][0] + MOVES[act][0], cur[i][1] + MOVES[act][1]
        prop.append((x, y) if (0 <= x < W and 0 <= y < H and not grid[x, y]) else cur[i])
    owner = {c: i for i, c in enumerate(cur)}
    for _ in range(A):
        first = {}
        for i, c in enumerate(prop):
            if c not in first:
                first[c] = i
        rejected = []
        for i in range(A):
            if prop[i] == cur[i]:
                continue
            o = owner.get(prop[i])
            m = first[prop[i]]
            hit = False
            if o is not None and o != i:
                hit = (prop[o] == cur[i]) or (prop[o] == cur[o])
            if not hit and m < i:
                hit = True
            if hit:
                rejected.append(i)
        if not rejected:
            break
        for i in rejected:
            prop[i] = cur[i]
    new_arrived = [bool(arrived[i]) or prop[i] == (int(goals[i][0]), int(goals[i][1])) for i in range(A)]
    return prop, new_arrived


def _c_bfs(grid, goal):
    """The C oracle's BFS (same fields as bfs_cost): fills a goal cache fast
    outside the timed region on large maps."""
    from oracle.oracle import bfs_u16

    return bfs_u16(grid, goal)[0]


def run_stage_worker(args):
    """Worker body: `steps` resident steps (step + token build) of one stage.
    An optional sixth item `fast_fill` fills the goal cache before timing with
    the C BFS instead of the deque BFS (the same fields; untimed)."""
    grids, starts, goals, actions, steps = args[:5]
    fast_fill = len(args) > 5 and args[5]
    import time

    E, A = starts.shape[:2]
    builder = CachedTokenBuilder(grids, A, bfs=_c_bfs if fast_fill else bfs_cost)
    pos = starts.astype(np.int64).copy()
    arrived = np.zeros((E, A), bool)
    hist = np.full((E, A, 5), 5, np.uint16)

    def rows_now():
        r = np.zeros((E, A, 13), np.uint16)
        r[..., 0] = np.arange(E)[:, None]
        r[..., 1] = np.arange(A)[None, :]
        r[..., 2:4] = pos
        r[..., 4:6] = goals
        r[..., 8:13] = hist
        return r.reshape(E * A, 13)

    builder.build(rows_now())  # first build: every goal is fresh (untimed cache fill)
    builder.bfs = bfs_cost
    t0 = time.perf_counter()
    for s in range(steps):
        tokens, _, active = builder.build(rows_now())
        act = actions[s]
        hist[..., :4] = hist[..., 1:]
        hist[..., 4] = np.where(active.reshape(E, A), act, 0)
        for e in range(E):
            new_pos, new_arr = resolve_step(grids[e], pos[e], goals[e], arrived[e], act[e])
            pos[e] = new_pos
            arrived[e] = new_arr
    return time.perf_counter() - t0, E * A * steps


def run_magat_worker(args):
    """Worker body: `steps` stateful MAGAT steps of one stage (step, occupancy
    refresh, nodes, edges; goals are fixed in standard_mapf, so no energy
    refresh after the first) with the C restatement, oracle/jl_oracle.c."""
    grids, starts, goals, actions, steps = args
    import time

    from oracle.oracle import OracleMagat, OracleSim

    E, A = starts.shape[:2]
    osim = OracleSim(grids, A, task_mode=1, max_episode_steps=1 << 30)
    osim.load_state(starts, goals)
    m = OracleMagat(grids, A)
    rows = osim.state_packed.copy()
    rows[:, 7] = 1
    m.update_energy(rows, len(rows))  # every goal fresh (untimed)
    t0 = time.perf_counter()
    for s in range(steps):
        osim.step(actions[s])
        m.refresh(osim.state_packed)
        m.nodes()
        m.edges()
    return time.perf_counter() - t0, E * A * steps


def run_fresh_worker(args):
    """Worker body: `builds` builds of one stage with every goal fresh (the
    goal caches cleared first), timed; returns (seconds, agents built)."""
    grids, starts, goals, builds = args
    import time

    E, A = starts.shape[:2]
    rows = np.zeros((E, A, 13), np.uint16)
    rows[..., 0] = np.arange(E)[:, None]
    rows[..., 1] = np.arange(A)[None, :]
    rows[..., 2:4] = starts
    rows[..., 4:6] = goals
    rows[..., 8:13] = 5
    rows = rows.reshape(E * A, 13)
    builder = CachedTokenBuilder(grids, A)
    t0 = time.perf_counter()
    for _ in range(builds):
        builder.goals = [None] * E  # every goal fresh
        builder.build(rows)
    return time.perf_counter() - t0, E * A * builds


def run_stage_build_worker(args):
    """Worker body of the frozen-record consumer on the host: the cached
    builder over `stages` stages of rows (positions change, goals fixed in the
    episode; goal cache filled before timing with the C BFS), timed; returns
    (seconds, agents built)."""
    grids, positions, goals = args
    import time

    S, E, A = positions.shape[:3]
    builder = CachedTokenBuilder(grids, A, bfs=_c_bfs)

    def rows(s):
        r = np.zeros((E, A, 13), np.uint16)
        r[..., 0] = np.arange(E)[:, None]
        r[..., 1] = np.arange(A)[None, :]
        r[..., 2:4] = positions[s]
        r[..., 4:6] = goals
        r[..., 8:13] = 5
        return r.reshape(E * A, 13)

    builder.build(rows(0))  # untimed cache fill
    builder.bfs = bfs_cost
    t0 = time.perf_counter()
    for s in range(1, S):
        builder.build(rows(s))
    return time.perf_counter() - t0, E * A * (S - 1)
