"""Seeded synthetic workloads for the benchmark configurations.

All generators take a ``numpy.random.Generator`` and return plain numpy
arrays in the reference layout: grids are uint8 [W, H] with 1 = obstacle,
x = row, y = column (grid_world_simulator.cpp:184-187).

* ``iid_grid``: i.i.d. obstacles at a density, then only the largest
  4-connected free component is kept free.
* ``maze_grid``: recursive-backtracker maze with corridors of width 1 or 2.
* ``warehouse_grid``: rectangular shelf blocks separated by 2-wide aisles.
* ``place_agents``: distinct starts and distinct goals drawn from the free
  cells, the validity rule of host_inputs.py:29-35.
"""
from __future__ import annotations

from collections import deque

import numpy as np


def largest_component(free: np.ndarray) -> np.ndarray:
    """Boolean mask of the largest 4-connected component of ``free``."""
    W, H = free.shape
    label = np.full((W, H), -1, dtype=np.int64)
    best_label, best_size, current = -1, 0, 0
    for sx in range(W):
        for sy in range(H):
            if not free[sx, sy] or label[sx, sy] >= 0:
                continue
            size = 0
            queue = deque([(sx, sy)])
            label[sx, sy] = current
            while queue:
                x, y = queue.popleft()
                size += 1
                for nx, ny in ((x - 1, y), (x + 1, y), (x, y - 1), (x, y + 1)):
                    if 0 <= nx < W and 0 <= ny < H and free[nx, ny] and label[nx, ny] < 0:
                        label[nx, ny] = current
                        queue.append((nx, ny))
            if size > best_size:
                best_label, best_size = current, size
            current += 1
    return label == best_label


def iid_grid(rng: np.random.Generator, W: int, H: int, density: float) -> np.ndarray:
    obstacles = rng.random((W, H)) < density
    keep = largest_component(~obstacles)
    return (~keep).astype(np.uint8)


def maze_grid(rng: np.random.Generator, W: int, H: int) -> np.ndarray:
    """Recursive-backtracker maze; each corridor of the spanning tree is 1 or 2 cells wide."""
    grid = np.ones((W, H), dtype=np.uint8)
    cw, ch = (W - 1) // 3, (H - 1) // 3  # 3-cell pitch: 2 cells of corridor + 1 of wall
    width = rng.integers(1, 3, size=(cw, ch))

    def carve_cell(cx, cy):
        x0, y0 = 1 + 3 * cx, 1 + 3 * cy
        w = int(width[cx, cy])
        grid[x0:x0 + w, y0:y0 + w] = 0

    def carve_link(a, b):
        (ax, ay), (bx, by) = a, b
        x0, y0 = 1 + 3 * min(ax, bx), 1 + 3 * min(ay, by)
        w = int(min(width[ax, ay], width[bx, by]))
        if ax != bx:
            grid[x0:x0 + 4, y0:y0 + w] = 0
        else:
            grid[x0:x0 + w, y0:y0 + 4] = 0

    visited = np.zeros((cw, ch), dtype=bool)
    start = (int(rng.integers(cw)), int(rng.integers(ch)))
    stack = [start]
    visited[start] = True
    carve_cell(*start)
    while stack:
        cx, cy = stack[-1]
        options = [
            (cx + dx, cy + dy)
            for dx, dy in ((-1, 0), (1, 0), (0, -1), (0, 1))
            if 0 <= cx + dx < cw and 0 <= cy + dy < ch and not visited[cx + dx, cy + dy]
        ]
        if not options:
            stack.pop()
            continue
        nxt = options[int(rng.integers(len(options)))]
        visited[nxt] = True
        carve_cell(*nxt)
        carve_link((cx, cy), nxt)
        stack.append(nxt)
    keep = largest_component(grid == 0)
    return (~keep).astype(np.uint8)


def warehouse_grid(W: int, H: int, *, shelf=(2, 8), aisle=2, margin=2) -> np.ndarray:
    """Shelf blocks of ``shelf`` cells separated by ``aisle``-wide aisles."""
    grid = np.zeros((W, H), dtype=np.uint8)
    sx, sy = shelf
    x = margin
    while x + sx <= W - margin:
        y = margin
        while y + sy <= H - margin:
            grid[x:x + sx, y:y + sy] = 1
            y += sy + aisle
        x += sx + aisle
    keep = largest_component(grid == 0)
    return (~keep).astype(np.uint8)


def place_agents(rng: np.random.Generator, grid: np.ndarray, n_agents: int):
    """Distinct starts and distinct goals (int16 [A, 2] each) on free cells."""
    free = np.argwhere(grid == 0)
    if len(free) < n_agents:
        raise ValueError("not enough free cells for the agents")
    starts = free[rng.choice(len(free), size=n_agents, replace=False)]
    goals = free[rng.choice(len(free), size=n_agents, replace=False)]
    return starts.astype(np.int16), goals.astype(np.int16)


def random_actions(rng: np.random.Generator, steps: int, n_envs: int, n_agents: int) -> np.ndarray:
    """Uniform actions in {wait, up, down, left, right}: uint8 [steps, E, A]."""
    return rng.integers(0, 5, size=(steps, n_envs, n_agents), dtype=np.uint8)


def make_batch(seed: int, n_envs: int, W: int, H: int, n_agents: int, kind: str = "iid",
               density: float = 0.2):
    """Grids uint8 [E, W, H] + starts/goals int16 [E, A, 2] for one configuration."""
    rng = np.random.default_rng(seed)
    grids = np.empty((n_envs, W, H), dtype=np.uint8)
    starts = np.empty((n_envs, n_agents, 2), dtype=np.int16)
    goals = np.empty((n_envs, n_agents, 2), dtype=np.int16)
    for e in range(n_envs):
        if kind == "iid":
            g = iid_grid(rng, W, H, density)
        elif kind == "maze":
            g = maze_grid(rng, W, H)
        elif kind == "warehouse":
            g = warehouse_grid(W, H)
        else:
            raise ValueError(f"unknown map kind {kind!r}")
        grids[e] = g
        starts[e], goals[e] = place_agents(rng, g, n_agents)
    return grids, starts, goals
