"""Seeded compact expert records shaped like the reference producers' output:
distinct free-cell positions and goals per env, episodes of random length
per env (a new episode brings new goals), uniform actions."""
from __future__ import annotations

import numpy as np

from iclr_2027_jointoom_amd.synthetic import make_batch


def make_compact(seed: int, E: int, W: int, A: int, S: int, mean_episode: float = 6.0):
    """grids uint8 [E, W, W] and (positions, actions, episode_starts, goals)."""
    grids, starts, goals0 = make_batch(seed, E, W, W, A)
    rng = np.random.default_rng(seed + 1)
    positions = np.zeros((S, E * A, 2), np.uint16)
    actions = rng.integers(0, 5, size=(S, E * A)).astype(np.uint8)
    episode_starts = (rng.random((S, E)) < 1.0 / mean_episode).astype(np.uint8)
    episode_starts[0] = 1
    pos = starts.astype(np.int64)
    goal_blocks = []
    for s in range(S):
        positions[s] = pos.reshape(E * A, 2)
        for e in np.flatnonzero(episode_starts[s]):
            # a rolled goal set stays distinct and on the env's free cells
            goal_blocks.append(np.roll(goals0[e], int(rng.integers(0, A)), axis=0).astype(np.uint16))
        pos = np.roll(pos, 1, axis=1)
    goals = np.stack(goal_blocks) if goal_blocks else np.zeros((0, A, 2), np.uint16)
    return grids, (positions, actions, episode_starts, goals)
