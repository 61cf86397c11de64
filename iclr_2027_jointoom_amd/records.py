"""Compact frozen expert records: 5 bytes per agent and step on disk and on
the host link, full 8/13-column stage rows rebuilt on the device.

The reference's frozen archives (frozen_stage_source.py:23-59) hold every
stage as uint16 rows, 16 B (MAGAT, 8 columns) or 26 B (MAPF-GPT, 13 columns)
per agent and step, and stream them row for row through the host ring.  The
producers that write those rows (mapf_gpt_online.py:215-258,
mapf_gpt_schema.py:43-66 and 118-126; topology_async.py:90-102 and 235-278)
fix most columns:

* env and agent ids are the row's place in the env-major stage;
* the refresh flag is 1 for every agent of an env whose episode starts at the
  stage (``initial_refresh_flags``) and 0 otherwise (``no_refresh_flags``);
* goals change only when an episode starts;
* the 5 history columns are the env's previous actions of the running
  episode, oldest first, 5 when there are none yet (``ActionHistory``).

A compact archive keeps only what is not implied::

    grids.npy           uint8  [E, H, W]    as save_records writes it
    positions.npy       uint16 [S, E*A, 2]  x, y of every agent at every stage
    actions.npy         uint8  [S, E*A]     the action taken at the stage
    episode_starts.npy  uint8  [S, E]       1 = env e starts an episode (all 1 at s = 0)
    goals.npy           uint16 [K, A, 2]    goals of the K episode starts, in (stage, env) order
    manifest.json       schema_version 1, format "compact", backend, agents, stages,
                        features, metadata, sha256 of every .npy

``save_compact_records`` takes the same stage rows as ``save_records`` and
refuses rows these rules do not produce, so expanding the archive gives back
exactly the rows it was made from.  ``RecordExpander`` rebuilds a stage's rows
on the device with ``jl_expand_records`` (include/jointloom.h).
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass
from pathlib import Path

import numpy as np

COMPACT_FORMAT = "compact"
EMPTY_ACTION = 5
HISTORY_LEN = 5
_FILES = ("grids.npy", "positions.npy", "actions.npy", "episode_starts.npy", "goals.npy")


def _features(backend: str) -> int:
    return 8 if backend == "magat" else 13


@dataclass
class CompactRecords:
    """The arrays of a compact archive (memory-mapped when loaded)."""

    positions: np.ndarray       # uint16 [S, N, 2]
    actions: np.ndarray         # uint8  [S, N]
    episode_starts: np.ndarray  # uint8  [S, E]
    goals: np.ndarray           # uint16 [K, A, 2]

    def __post_init__(self):
        starts = np.asarray(self.episode_starts, dtype=np.int64).reshape(-1)
        # index into goals of every (stage, env) that starts an episode
        self.goal_index = (np.cumsum(starts) - 1).reshape(self.episode_starts.shape)

    @property
    def num_stages(self) -> int:
        return int(self.positions.shape[0])

    @property
    def num_envs(self) -> int:
        return int(self.episode_starts.shape[1])

    @property
    def agents(self) -> int:
        return int(self.positions.shape[1] // self.num_envs)

    def env_goals(self, stage: int, env: int) -> np.ndarray | None:
        """Goals [A, 2] of the episode env starts at stage, or None."""
        if not self.episode_starts[stage, env]:
            return None
        return self.goals[int(self.goal_index[stage, env])]


def compact_from_stages(stages, num_envs: int, features: int) -> CompactRecords:
    """Compact records of full stage rows [S, E*A, F]; ValueError if the rows
    are not the ones the reference's producers write (module docstring)."""
    stages = np.asarray(stages)
    if stages.ndim != 3 or stages.shape[2] != features or stages.shape[1] % num_envs:
        raise ValueError("invalid stage archive")
    S, N, F = stages.shape
    A = N // num_envs
    blocks = stages.reshape(S, num_envs, A, F)
    if not np.array_equal(blocks[:, :, :, 0], np.broadcast_to(np.arange(num_envs)[None, :, None], (S, num_envs, A))):
        raise ValueError("stage environment order mismatch")
    if not np.array_equal(blocks[:, :, :, 1], np.broadcast_to(np.arange(A)[None, None, :], (S, num_envs, A))):
        raise ValueError("stage agent order mismatch")
    if np.any(stages[:, :, 6] > 4):
        raise ValueError("invalid action or refresh flag")
    refresh = blocks[:, :, :, 7]
    if np.any(refresh > 1):
        raise ValueError("invalid action or refresh flag")
    starts = refresh[:, :, 0]
    if np.any(refresh != starts[:, :, None]):
        raise ValueError("compact records need one refresh flag per env and stage "
                         "(all agents of an env start their episode together)")
    if not np.all(starts[0] == 1):
        raise ValueError("compact records need every env to start an episode at stage 0")
    goals_all = blocks[:, :, :, 4:6]
    same = np.all(goals_all[1:] == goals_all[:-1], axis=(2, 3))
    if np.any(~same & (starts[1:] == 0)):
        raise ValueError("compact records need goals that change only at an episode start")
    if features == 13:
        history = np.full((num_envs, A, HISTORY_LEN), EMPTY_ACTION, np.uint16)
        for s in range(S):
            history[starts[s] == 1] = EMPTY_ACTION
            if not np.array_equal(blocks[s, :, :, 8:13], history):
                raise ValueError(f"stage {s}: history columns are not the previous actions of the episode")
            history[:, :, :-1] = history[:, :, 1:]
            history[:, :, -1] = blocks[s, :, :, 6]
    s_idx, e_idx = np.nonzero(starts)
    return CompactRecords(
        positions=np.ascontiguousarray(stages[:, :, 2:4]).astype(np.uint16),
        actions=stages[:, :, 6].astype(np.uint8),
        episode_starts=starts.astype(np.uint8),
        goals=np.ascontiguousarray(goals_all[s_idx, e_idx]).astype(np.uint16),
    )


def validate_compact(records: CompactRecords, grids, agents: int) -> None:
    """The checks validate_stage (host_inputs.py:17-36) makes of full rows,
    on compact records: actions, flags, coordinates inside the map, off
    obstacles and distinct within an env, for positions and for goals."""
    grids = np.asarray(grids)
    E = len(grids)
    S = records.num_stages
    N = E * agents
    if records.positions.shape != (S, N, 2) or records.actions.shape != (S, N):
        raise ValueError("record shape differs from manifest")
    if records.episode_starts.shape != (S, E) or records.goals.shape[1:] != (agents, 2):
        raise ValueError("record shape differs from manifest")
    starts = np.asarray(records.episode_starts)
    if np.any(starts > 1) or (S and not np.all(starts[0] == 1)):
        raise ValueError("invalid action or refresh flag")
    if int(starts.sum()) != records.goals.shape[0]:
        raise ValueError("record shape differs from manifest")
    occupied = np.asarray(grids, dtype=bool)
    d0, d1 = occupied.shape[1], occupied.shape[2]
    env_of = np.repeat(np.arange(E, dtype=np.int64), agents)

    def check(coords: np.ndarray, envs: np.ndarray, groups: int) -> None:
        x = coords[:, 0].astype(np.int64)
        y = coords[:, 1].astype(np.int64)
        if np.any(x >= d0) or np.any(y >= d1):
            raise ValueError("coordinates outside map")
        if np.any(occupied[envs, x, y]):
            raise ValueError("coordinates on obstacles")
        cells = np.sort((np.repeat(np.arange(groups, dtype=np.int64), agents) * (d0 * d1)) + x * d1 + y)
        if np.any(cells[1:] == cells[:-1]):
            raise ValueError("duplicate joint positions or goals")

    for s in range(S):
        if np.any(records.actions[s] > 4):
            raise ValueError("invalid action or refresh flag")
        check(np.asarray(records.positions[s]), env_of, E)
    if records.goals.shape[0]:
        _, goal_env = np.nonzero(starts)
        g = np.asarray(records.goals).reshape(-1, 2)
        check(g, np.repeat(goal_env, agents), records.goals.shape[0])


def _sha256(path) -> str:
    from .ring import sha256_file

    return sha256_file(path)


def write_compact_records(output, *, backend: str, grids, records: CompactRecords, metadata) -> dict:
    """Write a compact archive directory (module docstring) and its manifest."""
    output = Path(output)
    grids = np.asarray(grids, dtype=np.uint8)
    agents = records.agents
    validate_compact(records, grids, agents)
    output.mkdir(parents=True, exist_ok=False)
    np.save(output / "grids.npy", grids, allow_pickle=False)
    np.save(output / "positions.npy", np.ascontiguousarray(records.positions, dtype=np.uint16), allow_pickle=False)
    np.save(output / "actions.npy", np.ascontiguousarray(records.actions, dtype=np.uint8), allow_pickle=False)
    np.save(output / "episode_starts.npy", np.ascontiguousarray(records.episode_starts, dtype=np.uint8),
            allow_pickle=False)
    np.save(output / "goals.npy", np.ascontiguousarray(records.goals, dtype=np.uint16), allow_pickle=False)
    manifest = dict(schema_version=1, format=COMPACT_FORMAT, backend=backend, agents=agents,
                    stages=records.num_stages, features=_features(backend), goal_blocks=int(records.goals.shape[0]),
                    metadata=metadata, hashes={name: _sha256(output / name) for name in _FILES})
    (output / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest


def save_compact_records(output, *, backend, grids, stages, metadata) -> dict:
    """save_records (frozen_stage_source.py:23-42) with the compact layout:
    same arguments, same rejections, 5 bytes per agent and step."""
    stages = np.asarray(stages)
    if not np.issubdtype(stages.dtype, np.integer) or np.any(stages < 0) or np.any(stages > 65535):
        raise ValueError("records must contain uint16-representable integers")
    stages = stages.astype(np.uint16)
    features = _features(backend)
    if stages.ndim != 3 or not len(stages) or stages.shape[1] % len(grids):
        raise ValueError("invalid stage archive")
    records = compact_from_stages(stages, len(grids), features)
    return write_compact_records(output, backend=backend, grids=grids, records=records, metadata=metadata)


def is_compact_archive(root) -> bool:
    m = json.loads((Path(root) / "manifest.json").read_text())
    return m.get("format") == COMPACT_FORMAT


def load_compact_records(root):
    """Verify hashes, shapes and contents; arrays are memory-mapped
    (load_records, frozen_stage_source.py:45-59, for the compact layout)."""
    root = Path(root)
    m = json.loads((root / "manifest.json").read_text())
    if (m.get("schema_version") != 1 or m.get("format") != COMPACT_FORMAT
            or set(m.get("hashes", {})) != set(_FILES)):
        raise ValueError("unsupported or incomplete record manifest")
    for name, expected in m["hashes"].items():
        if _sha256(root / name) != expected:
            raise ValueError(f"record hash mismatch: {name}")
    grids = np.load(root / "grids.npy", allow_pickle=False)
    arrays = {name[:-4]: np.load(root / name, mmap_mode="r", allow_pickle=False) for name in _FILES[1:]}
    records = CompactRecords(**arrays)
    if records.num_stages != m["stages"] or m["features"] != _features(m["backend"]):
        raise ValueError("record shape differs from manifest")
    validate_compact(records, grids, m["agents"])
    return m, grids, records


class RecordExpander:
    """Device state and launcher of ``jl_expand_records``: the running goals
    and histories of every agent, carried from one expanded stage to the
    next.  Stages must be expanded in order on one stream."""

    def __init__(self, num_envs: int, agents: int, features: int, device="cuda:0"):
        import torch

        from ._abi import RecordsDesc, load_library

        if features not in (8, 13):
            raise ValueError(f"features must be 8 or 13, got {features}")
        if num_envs <= 0 or agents <= 0:
            raise ValueError("num_envs and agents must be positive")
        self._lib = load_library()
        self.device = torch.device(device)
        self.num_envs, self.agents, self.features = int(num_envs), int(agents), int(features)
        n = self.num_envs * self.agents
        self.goals = torch.zeros((n, 2), dtype=torch.int16, device=self.device)
        self.history = torch.zeros((n, 8), dtype=torch.uint8, device=self.device)
        self._desc = RecordsDesc(n_envs=self.num_envs, n_agents=self.agents, features=self.features)
        self._desc.goals = self.goals.data_ptr()
        self._desc.history = self.history.data_ptr()

    def expand(self, positions, actions, episode_start, new_goals, rows, stream=None) -> None:
        """rows[N, F] <- the stage (device tensors: positions [N,2] 16-bit,
        actions [N] uint8, episode_start [E] uint8, new_goals [N,2] 16-bit)."""
        import torch

        from ._abi import check

        n = self.num_envs * self.agents
        for name, t, shape in (("positions", positions, (n, 2)), ("actions", actions, (n,)),
                               ("episode_start", episode_start, (self.num_envs,)),
                               ("new_goals", new_goals, (n, 2)), ("rows", rows, (n, self.features))):
            if t.device != self.device or not t.is_contiguous():
                raise RuntimeError(f"{name} must be a contiguous tensor on {self.device}")
            if t.numel() != int(np.prod(shape)):
                raise RuntimeError(f"{name} shape must be {list(shape)}, got {list(t.shape)}")
        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        d = self._desc
        d.positions = positions.data_ptr()
        d.actions = actions.data_ptr()
        d.episode_start = episode_start.data_ptr()
        d.new_goals = new_goals.data_ptr()
        d.rows = rows.data_ptr()
        check(self._lib.jl_expand_records(ctypes.byref(d), stream.cuda_stream), "jl_expand_records")

    def expand_ptrs(self, positions: int, actions: int, episode_start: int, new_goals: int, rows: int,
                    stream_handle: int) -> None:
        """expand() on raw device addresses (the ring's staging slots)."""
        from ._abi import check

        d = self._desc
        d.positions, d.actions, d.episode_start, d.new_goals, d.rows = (
            positions, actions, episode_start, new_goals, rows)
        check(self._lib.jl_expand_records(ctypes.byref(d), stream_handle), "jl_expand_records")
