"""CPU restatement of the rows the reference's expert producers write, from
compact records (the checker of jl_expand_records and of the compact
archive encoder).

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py as the checker;
the product path (iclr_2027_jointoom_amd) never imports it.

Follows, per env and stage:
* mapf_gpt_expert_worker_loop, mapf_gpt_online.py:215-258: rows are built
  from the observation and the action, the action is recorded into the
  history after the rows are written, and an episode end resets the history
  and sets the refresh flags of the next stage to 1 (else 0);
* ActionHistory, mapf_gpt_schema.py:43-66: five slots, oldest first, filled
  with 5 (the empty action); append shifts left and writes the newest last;
* build_mapf_gpt_rows, mapf_gpt_schema.py:118-126: columns env, agent, x, y,
  goal x, goal y, action, refresh flag, history[0..4];
* _build_step_data, topology_async.py:90-102 with the MAGAT loop :246-278:
  the same first 8 columns, refresh flags 1 at an episode start, else 0.

Pinned by the reference's own known answers (tests/test_records.py):
test_mapf_gpt_schema.py:12-28 and test_mapf_gpt_online.py:19-45 for the
history rule, test_pipeline.py:558-574 for the 8-column layout.
"""
from __future__ import annotations

import numpy as np

EMPTY_ACTION = 5


class History:
    """Five previous actions per agent, oldest first (mapf_gpt_schema.py:43-66)."""

    def __init__(self, agents: int):
        self.slots = [[EMPTY_ACTION] * 5 for _ in range(agents)]

    def snapshot(self) -> list[list[int]]:
        return [list(s) for s in self.slots]

    def append(self, actions) -> None:
        for s, a in zip(self.slots, actions):
            del s[0]
            s.append(int(a))

    def reset(self) -> None:
        for s in self.slots:
            s[:] = [EMPTY_ACTION] * 5


def expand_records(positions, actions, episode_starts, goals, num_envs: int, features: int) -> np.ndarray:
    """Full stage rows uint16 [S, E*A, F] of compact records.

    positions [S, E*A, 2], actions [S, E*A], episode_starts [S, E] and goals
    [K, A, 2] (the goals of the K episode starts in (stage, env) order)."""
    positions = np.asarray(positions)
    S, N = positions.shape[:2]
    A = N // num_envs
    out = np.zeros((S, N, features), np.uint16)
    histories = [History(A) for _ in range(num_envs)]
    current = [None] * num_envs
    k = 0
    for s in range(S):
        for e in range(num_envs):
            start = int(episode_starts[s][e])
            if start:
                histories[e].reset()
                current[e] = np.asarray(goals[k])
                k += 1
            hist = histories[e].snapshot()
            acts = [int(actions[s][e * A + a]) for a in range(A)]
            for a in range(A):
                row = [e, a, int(positions[s][e * A + a][0]), int(positions[s][e * A + a][1]),
                       int(current[e][a][0]), int(current[e][a][1]), acts[a], start]
                if features == 13:
                    row += hist[a]
                out[s, e * A + a] = row
            histories[e].append(acts)
    return out
