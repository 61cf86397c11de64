"""numpy front-end of the C oracle (oracle/jl_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product path
(iclr_2027_jointoom_amd) never imports it.

The host-side state classes hold numpy arrays with the same shapes, dtypes
and meaning as the GPU simulator / builders and drive the C functions
through the same descriptor structs (with host pointers).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

from iclr_2027_jointoom_amd._abi import MagatDesc, MapfGPTDesc, SimDesc

ORACLE_DIR = Path(__file__).resolve().parent
# JLO_SANITIZE=1: the AddressSanitizer + UBSan build (`make -C oracle sanitize`;
# the interpreter needs the ASan runtime preloaded, see `make check-sanitize`)
SANITIZE = os.environ.get("JLO_SANITIZE") == "1"
LIB_PATH = ORACLE_DIR / ("libjl_oracle_asan.so" if SANITIZE else "libjl_oracle.so")
_LIB = None


def build() -> Path:
    target = ["sanitize"] if SANITIZE else []
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), *target], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, i32 = ctypes.c_void_p, ctypes.c_int
        L.jlo_encode_map.argtypes = [vp, vp, i32, i32, i32]
        L.jlo_resolve_env.argtypes = [vp, i32, i32, i32, vp, vp, vp, vp, vp, i32]
        L.jlo_step.argtypes = [ctypes.POINTER(SimDesc), i32]
        L.jlo_load_state.argtypes = [ctypes.POINTER(SimDesc), vp, vp, vp, vp]
        L.jlo_bfs_u16.argtypes = [vp, i32, i32, i32, i32, vp, vp]
        L.jlo_bfs_u16.restype = i32
        L.jlo_energy_u8.argtypes = [vp, i32, i32, i32, i32, vp]
        L.jlo_energy_maps.argtypes = [vp, vp, vp, i32, i32, i32, i32, i32, i32]
        for name in ("jlo_mapfgpt_bfs", "jlo_mapfgpt_tokens"):
            getattr(L, name).argtypes = [ctypes.POINTER(MapfGPTDesc)]
        L.jlo_mapfgpt_unpack_rows.argtypes = [ctypes.POINTER(MapfGPTDesc), vp]
        L.jlo_mapfgpt_build_rows.argtypes = [ctypes.POINTER(MapfGPTDesc), vp]
        L.jlo_mapfgpt_unpack_state.argtypes = [ctypes.POINTER(MapfGPTDesc), vp, vp, vp, vp]
        L.jlo_mapfgpt_build_state.argtypes = [ctypes.POINTER(MapfGPTDesc), vp, vp, vp, vp]
        L.jlo_mapfgpt_append.argtypes = [ctypes.POINTER(MapfGPTDesc), vp]
        for name in ("jlo_magat_occupancy", "jlo_magat_nodes", "jlo_magat_edges"):
            getattr(L, name).argtypes = [ctypes.POINTER(MagatDesc)]
        u64 = ctypes.c_uint64
        L.jlo_splitmix64.argtypes = [u64]
        L.jlo_splitmix64.restype = u64
        L.jlo_xorshift64s.argtypes = [ctypes.POINTER(u64)]
        L.jlo_xorshift64s.restype = u64
        L.jlo_seed_rng.argtypes = [vp, ctypes.c_int64, u64]
        L.jlo_free_cells.argtypes = [ctypes.POINTER(SimDesc), vp, vp, vp, vp]
        L.jlo_init_agents.argtypes = [ctypes.POINTER(SimDesc), vp, vp, vp]
        _LIB = L
    return _LIB


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags.c_contiguous
    return a.ctypes.data


def encode(grids: np.ndarray) -> np.ndarray:
    """int/uint8 [E, W, H] obstacle grids -> uint32 [E, W*H/32] bitmaps."""
    g = np.ascontiguousarray(grids, dtype=np.int32)
    E, W, H = g.shape
    bits = np.zeros((E, W * H // 32), dtype=np.uint32)
    lib().jlo_encode_map(_p(g), _p(bits), E, W, H)
    return bits


def resolve_env(grid: np.ndarray, cur: np.ndarray, arrived, actions, naive: bool = False):
    """One env: final int32 [A, 2] positions and uint8 [A] outcome categories."""
    W, H = grid.shape
    bits = encode(grid[None])[0]
    cur = np.ascontiguousarray(cur, dtype=np.int32)
    A = cur.shape[0]
    arr = np.ascontiguousarray(np.zeros(A, np.uint8) if arrived is None else arrived, dtype=np.uint8)
    act = np.ascontiguousarray(actions, dtype=np.uint8)
    out = np.zeros((A, 2), dtype=np.int32)
    cat = np.zeros(A, dtype=np.uint8)
    lib().jlo_resolve_env(_p(bits), W, H, A, _p(cur), _p(arr), _p(act), _p(out), _p(cat), int(naive))
    return out, cat


def bfs_u16(grid: np.ndarray, goal) -> tuple[np.ndarray, int, int]:
    """(uint16 [W, H] field, bad_goal flag, overflow count)."""
    W, H = grid.shape
    bits = encode(grid[None])[0]
    out = np.zeros((W, H), dtype=np.uint16)
    overflow = ctypes.c_int(0)
    bad = lib().jlo_bfs_u16(_p(bits), W, H, int(goal[0]), int(goal[1]), _p(out), ctypes.byref(overflow))
    return out, int(bad), int(overflow.value)


def energy_u8(grid: np.ndarray, goal) -> np.ndarray:
    W, H = grid.shape
    bits = encode(grid[None])[0]
    out = np.zeros((W, H), dtype=np.uint8)
    lib().jlo_energy_u8(_p(bits), W, H, int(goal[0]), int(goal[1]), _p(out))
    return out


class OracleSim:
    """Host mirror of GridWorldSimulator state for standard_mapf stepping."""

    def __init__(self, grids: np.ndarray, n_agents: int, task_mode: int = 1, max_episode_steps: int = 256):
        grids = np.asarray(grids)
        E, W, H = grids.shape
        A = int(n_agents)
        self.E, self.A, self.W, self.H = E, A, W, H
        self.grid_bits = encode(grids)
        self.grid_ocp = np.zeros_like(self.grid_bits)
        self.cur_x = np.zeros((E, A), np.uint16)
        self.cur_y = np.zeros((E, A), np.uint16)
        self.goal_x = np.zeros((E, A), np.uint16)
        self.goal_y = np.zeros((E, A), np.uint16)
        self.actions = np.zeros((E, A), np.uint8)
        self.arrived = np.zeros((E, A), np.uint8)
        self.goal_changed = np.zeros((E, A), np.uint8)
        self.rewards = np.zeros((E, A), np.float32)
        self.terminated = np.zeros(E, np.uint8)
        self.truncated = np.zeros(E, np.uint8)
        self.step_counts = np.zeros(E, np.int32)
        self.state_packed = np.zeros((E * A, 8), np.uint16)
        self.outcomes = np.zeros((E, A), np.uint8)
        self.desc = SimDesc(
            n_envs=E, n_agents=A, map_w=W, map_h=H, task_mode=task_mode,
            max_episode_steps=max_episode_steps,
            grid_bits=_p(self.grid_bits), grid_ocp=_p(self.grid_ocp),
            cur_x=_p(self.cur_x), cur_y=_p(self.cur_y), goal_x=_p(self.goal_x), goal_y=_p(self.goal_y),
            actions=_p(self.actions), arrived=_p(self.arrived), goal_changed=_p(self.goal_changed),
            rewards=_p(self.rewards), terminated=_p(self.terminated), truncated=_p(self.truncated),
            step_counts=_p(self.step_counts), state_packed=_p(self.state_packed),
            outcomes=_p(self.outcomes),
        )

    def load_state(self, positions, goals, arrived=None, step_counts=None) -> None:
        pos = np.ascontiguousarray(positions, dtype=np.int16)
        gol = np.ascontiguousarray(goals, dtype=np.int16)
        arr = np.ascontiguousarray(
            np.zeros((self.E, self.A)) if arrived is None else arrived, dtype=np.uint8)
        cnt = np.ascontiguousarray(np.zeros(self.E) if step_counts is None else step_counts, dtype=np.int32)
        lib().jlo_load_state(ctypes.byref(self.desc), _p(pos), _p(gol), _p(arr), _p(cnt))

    def seed_rng(self, seed: int) -> None:
        """init_rng: one xorshift64* state per agent (jlo_seed_rng)."""
        self.rng_state = np.zeros(self.E * self.A, np.uint64)
        lib().jlo_seed_rng(_p(self.rng_state), self.rng_state.size, int(seed) & 0xFFFFFFFFFFFFFFFF)
        self.desc.rng_state = _p(self.rng_state)

    def lifelong_init(self, extents=None) -> None:
        """run_initialization: free-cell lists inside the real extents, then
        random distinct starts and goals drawn from them; afterwards
        lifelong steps draw new goals from the same lists."""
        E, W, H = self.E, self.W, self.H
        ext = np.ascontiguousarray(
            np.tile([W, H], (E, 1)) if extents is None else extents, dtype=np.int32)
        self.free_cells = np.zeros(E * W * H, np.uint32)
        self.env_offsets = np.zeros(E, np.int32)
        self.env_counts = np.zeros(E, np.int32)
        lib().jlo_free_cells(ctypes.byref(self.desc), _p(ext), _p(self.free_cells), _p(self.env_offsets),
                             _p(self.env_counts))
        lib().jlo_init_agents(ctypes.byref(self.desc), _p(self.free_cells), _p(self.env_offsets),
                              _p(self.env_counts))
        d = self.desc
        d.free_cells = _p(self.free_cells)
        d.env_offsets = _p(self.env_offsets)
        d.env_counts = _p(self.env_counts)

    def set_goal_candidates(self, candidates, cells, counts) -> None:
        """Candidate lists of the deterministic lifelong mode (host copies)."""
        self.goal_candidates = np.ascontiguousarray(candidates, dtype=np.int32)
        self.candidate_cells = np.ascontiguousarray(cells, dtype=np.int16).view(np.uint16)
        self.candidate_counts = np.ascontiguousarray(counts, dtype=np.int32)
        self.goal_cursors = np.zeros((self.E, self.A), np.int32)
        d = self.desc
        d.goal_candidates = _p(self.goal_candidates)
        d.candidate_cells = _p(self.candidate_cells)
        d.candidate_counts = _p(self.candidate_counts)
        d.goal_cursors = _p(self.goal_cursors)
        d.candidate_length = self.goal_candidates.shape[2]
        d.candidate_stride = self.candidate_cells.shape[1]

    def step(self, actions=None, naive: bool = False) -> None:
        if actions is not None:
            self.actions[...] = actions
        lib().jlo_step(ctypes.byref(self.desc), int(naive))

    def positions(self) -> np.ndarray:
        return np.stack([self.cur_x, self.cur_y], axis=-1).astype(np.int16)


class OracleMapfGPT:
    """Host mirror of MapfGPTObservationBuilder."""

    def __init__(self, grids: np.ndarray, n_agents: int):
        grids = np.asarray(grids)
        E, W, H = grids.shape
        A = int(n_agents)
        N = E * A
        self.E, self.A, self.W, self.H = E, A, W, H
        self.grid_bits = encode(grids)
        self.state_packed = np.zeros((N, 8), np.uint16)
        self.histories = np.full((N, 5), 5, np.uint16)
        self.labels = np.zeros(N, np.int64)
        self.cost_to_go = np.full((E, A, W, H), 0xFFFF, np.uint16)
        self.agent_at_cell = np.full((E, W, H), -1, np.int32)
        self.goal_cache = np.full((N, 2), 0xFFFF, np.uint16)
        self.tokens = np.full((N, 256), 66, np.int32)
        self.active_mask = np.zeros(N, np.uint8)
        self.diagnostics = np.zeros(4, np.int32)
        self.desc = MapfGPTDesc(
            n_envs=E, n_agents=A, map_w=W, map_h=H, grid_bits=_p(self.grid_bits),
            state_packed=_p(self.state_packed), histories=_p(self.histories), labels=_p(self.labels),
            cost_to_go=_p(self.cost_to_go), agent_at_cell=_p(self.agent_at_cell),
            goal_cache=_p(self.goal_cache), tokens=_p(self.tokens), active_mask=_p(self.active_mask),
            diagnostics=_p(self.diagnostics),
        )

    def build_rows(self, rows) -> None:
        r = np.ascontiguousarray(rows, dtype=np.uint16)
        lib().jlo_mapfgpt_build_rows(ctypes.byref(self.desc), _p(r))

    def build_state(self, cur_x, cur_y, goal_x, goal_y) -> None:
        arrs = [np.ascontiguousarray(a, dtype=np.int16) for a in (cur_x, cur_y, goal_x, goal_y)]
        lib().jlo_mapfgpt_build_state(ctypes.byref(self.desc), *[_p(a) for a in arrs])

    def append(self, actions) -> None:
        a = np.ascontiguousarray(actions, dtype=np.uint8)
        lib().jlo_mapfgpt_append(ctypes.byref(self.desc), _p(a))


def energy_maps(grids, states, length, n_agents, incremental_only=False, energy=None) -> np.ndarray:
    grids = np.asarray(grids)
    E, W, H = grids.shape
    bits = encode(grids)
    if energy is None:
        energy = np.zeros((E, n_agents, W, H), np.uint8)
    st = np.ascontiguousarray(states, dtype=np.uint16)
    lib().jlo_energy_maps(_p(bits), _p(energy), _p(st), int(length), E, int(n_agents), W, H,
                          int(incremental_only))
    return energy


class OracleMagat:
    """Host mirror of the MAGAT builder buffers (stateless semantics)."""

    def __init__(self, grids: np.ndarray, n_agents: int):
        grids = np.asarray(grids)
        E, W, H = grids.shape
        A = int(n_agents)
        N = E * A
        self.E, self.A, self.W, self.H = E, A, W, H
        self.grid_bits = encode(grids)
        self.grid_ocp = np.zeros_like(self.grid_bits)
        self.energy = np.zeros((E, A, W, H), np.uint8)
        self.states = np.zeros((N, 8), np.uint16)
        self.pyg_x = np.zeros((N, 676), np.float32)
        self.pyg_pos = np.zeros((N, 2), np.float32)
        self.edge_counts = np.zeros(N, np.int32)
        self.edge_prefix = np.zeros(N + 1, np.int64)
        self.num_edges = np.zeros(1, np.int64)
        cap = E * A * A
        self.edge_index = np.zeros((2, cap), np.int64)
        self.edge_attr = np.zeros((cap, 3), np.float32)
        self.env_edge_base = np.zeros(E + 1, np.int64)
        self.desc = MagatDesc(
            n_envs=E, n_agents=A, map_w=W, map_h=H, grid_bits=_p(self.grid_bits),
            grid_ocp=_p(self.grid_ocp), energy=_p(self.energy), states=_p(self.states),
            pyg_x=_p(self.pyg_x), pyg_pos=_p(self.pyg_pos), edge_counts=_p(self.edge_counts),
            edge_prefix=_p(self.edge_prefix), num_edges=_p(self.num_edges),
            edge_index=_p(self.edge_index), edge_attr=_p(self.edge_attr), edge_capacity=cap,
            env_edge_base=_p(self.env_edge_base),
        )

    def refresh(self, states) -> None:
        """refresh_compact_state_from_raw_batch: fill -1, copy rows, rebuild occupancy."""
        st = np.asarray(states, dtype=np.uint16)
        self.states.fill(0xFFFF)
        self.states[: len(st)] = st
        self.grid_ocp.fill(0)
        lib().jlo_magat_occupancy(ctypes.byref(self.desc))

    def update_energy(self, states, length) -> None:
        st = np.ascontiguousarray(states, dtype=np.uint16)
        lib().jlo_energy_maps(_p(self.grid_bits), _p(self.energy), _p(st), int(length), self.E, self.A,
                              self.W, self.H, 0)

    def nodes(self) -> None:
        lib().jlo_magat_nodes(ctypes.byref(self.desc))

    def edges(self) -> None:
        lib().jlo_magat_edges(ctypes.byref(self.desc))

    def valid_edges(self):
        n = int(self.num_edges[0])
        return self.edge_index[:, :n], self.edge_attr[:n]
