"""Python mirror of the reference's ``grid_world_cpp`` extension module.

Same classes, constructor arguments, methods, read-only tensor attributes,
``memory_tensors`` dicts and error messages as the pybind11 surface in
/root/reference/src/cuda_backend/bind.cpp:94-237, backed by the gfx950 C ABI
of include/jointloom.h.  Every tensor is allocated once at construction on the
grid's device and attribute reads return that same tensor object, so callers
may mutate them in place; inputs are copied in.  All device work is enqueued
on the caller's current stream.

Map profile: the reference compiles one map size (MAPF_CUDA_MAP_PROFILE=WxH,
default 128x128, setup.py:9-40).  The kernels here take the size at run time
(H a multiple of 32 up to 256, W <= 256); ``profile(w, h)`` returns a module-like
namespace whose classes check grids against that size, and the module-level
classes use the size named by MAPF_CUDA_MAP_PROFILE.
"""
from __future__ import annotations

import ctypes
import os
import types

import torch

from ._abi import BUILD_SCRATCH_WORDS, GAVE_UP_WORD, MagatDesc, MapfGPTDesc, SimDesc, check, load_library, tiled_field_cells

TASK_LIFELONG = 0
TASK_STANDARD_MAPF = 1
# CostTracer steps (rebuttal/online-rl/native/src/cuda_backend/grid_world_cuda.h:44-46)
TASK_COSTTRACER = 2
_TASK_NAMES = {TASK_LIFELONG: "lifelong", TASK_STANDARD_MAPF: "standard_mapf", TASK_COSTTRACER: "costtracer"}
PYG_OBS_DIAM = 13
PYG_OBS_AREA = PYG_OBS_DIAM * PYG_OBS_DIAM
RADIUS = 5
_LEGACY_SMEM_LIMIT = 96 * 1024


def _require(cond: bool, message: str) -> None:
    """TORCH_CHECK equivalent: RuntimeError with the reference's message."""
    if not cond:
        raise RuntimeError(message)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The current stream of `device` as a raw handle (without building a
    torch Stream object, a few microseconds per call on the step path)."""
    if _RAW_STREAM is not None and device.index is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _parse_task_mode(mode: str) -> int:
    """grid_world_simulator.cpp:30-40 of rebuttal/online-rl/native/src/cuda_backend
    (the main tree's parser without "costtracer" has the same message)."""
    if mode == "costtracer":
        return TASK_COSTTRACER
    if mode == "lifelong":
        return TASK_LIFELONG
    if mode == "standard_mapf":
        return TASK_STANDARD_MAPF
    raise ValueError(
        f"Unknown task mode '{mode}'. Expected one of: lifelong, standard_mapf"
    )


_BUILDER_MODES = ("auto", "legacy_fullmap", "local_gather")
_GATHER_IMPLS = ("auto", "scalar", "async_sm89plus")


class _PygModeMixin:
    """Builder-mode properties (grid_world_simulator.cpp:16-160).

    Every mode runs the same gfx950 node kernel; the properties keep the
    reference's names, validation and resolution rules so callers that set or
    log them keep working.  The sm89 asynchronous-copy variant does not exist
    on this target, so ``async_sm89plus`` resolves to ``local_gather_scalar``.
    """

    _builder_mode = "auto"
    _gather_impl = "auto"

    def _legacy_supported(self) -> bool:
        smem = self._MAP_W * (self._MAP_H + 1) * 2 + 4 * self.n_agents * 2
        return (
            self._MAP_W == 128
            and self._MAP_H == 128
            and self.n_agents <= 256
            and smem <= _LEGACY_SMEM_LIMIT
        )

    @property
    def pyg_builder_mode(self) -> str:
        return self._builder_mode

    @pyg_builder_mode.setter
    def pyg_builder_mode(self, mode: str) -> None:
        if mode not in _BUILDER_MODES:
            raise ValueError(
                f"Unknown pyg builder mode '{mode}'. Expected one of: auto, legacy_fullmap, local_gather"
            )
        if mode == "legacy_fullmap" and not self._legacy_supported():
            raise RuntimeError(
                "legacy_fullmap builder mode requires n_agents <= 256 and shared memory usage within the legacy budget"
            )
        self._builder_mode = mode

    @property
    def pyg_local_gather_impl(self) -> str:
        return self._gather_impl

    @pyg_local_gather_impl.setter
    def pyg_local_gather_impl(self, mode: str) -> None:
        if mode not in _GATHER_IMPLS:
            raise ValueError(
                f"Unknown pyg local gather impl '{mode}'. Expected one of: auto, scalar, async_sm89plus"
            )
        self._gather_impl = mode

    @property
    def resolved_pyg_builder_impl(self) -> str:
        if self._builder_mode == "legacy_fullmap" or (
            self._builder_mode == "auto" and self._legacy_supported()
        ):
            return "legacy_fullmap"
        return "local_gather_scalar"


class _PygStorage:
    """PyG node/graph tensors shared by both simulators (bind.cpp:173-190)."""

    def _alloc_pyg(self, E: int, A: int, device: torch.device) -> None:
        N = E * A
        self.t_pyg_x = torch.zeros((N, 4 * PYG_OBS_AREA), dtype=torch.float32, device=device)
        self.t_pyg_pos = torch.zeros((N, 2), dtype=torch.float32, device=device)
        self.max_edges_per_env = A * A
        cap = E * self.max_edges_per_env
        self.t_edge_counts = torch.zeros((N,), dtype=torch.int32, device=device)
        self.t_pyg_edge_index_storage = torch.zeros((2, cap), dtype=torch.int64, device=device)
        self.t_pyg_edge_attr_storage = torch.zeros((cap, 3), dtype=torch.float32, device=device)
        self.t_pyg_edge_prefix = torch.zeros((N + 1,), dtype=torch.int64, device=device)
        self.t_pyg_num_edges = torch.zeros((1,), dtype=torch.int64, device=device)
        # the reference's CUB workspace: env bases [E + 1], then one edge
        # total per (env, 64-agent slice) from the node builder
        slices = (A + 63) // 64
        self.t_scan_temp_storage = torch.zeros((E + 1 + E * slices,), dtype=torch.int64, device=device)
        self.t_pyg_batch = torch.arange(E, dtype=torch.int64, device=device).repeat_interleave(A)
        self.t_pyg_ptr = torch.arange(E + 1, dtype=torch.int64, device=device) * A
        self.t_pyg_edge_index = self.t_pyg_edge_index_storage.narrow(1, 0, 0)
        self.t_pyg_edge_attr = self.t_pyg_edge_attr_storage.narrow(0, 0, 0)

    def _magat_desc(self, states: torch.Tensor, energy: torch.Tensor) -> MagatDesc:
        return MagatDesc(
            n_envs=self.n_envs,
            n_agents=self.n_agents,
            map_w=self._MAP_W,
            map_h=self._MAP_H,
            grid_bits=_ptr(self.t_grid_compressed),
            grid_ocp=_ptr(self.t_grid_ocp),
            energy=_ptr(energy),
            states=_ptr(states),
            pyg_x=_ptr(self.t_pyg_x),
            pyg_pos=_ptr(self.t_pyg_pos),
            edge_counts=_ptr(self.t_edge_counts),
            edge_prefix=_ptr(self.t_pyg_edge_prefix),
            num_edges=_ptr(self.t_pyg_num_edges),
            edge_index=_ptr(self.t_pyg_edge_index_storage),
            edge_attr=_ptr(self.t_pyg_edge_attr_storage),
            edge_capacity=int(self.t_pyg_edge_attr_storage.shape[0]),
            env_edge_base=_ptr(self.t_scan_temp_storage),
        )

    def _run_nodes(self) -> None:
        check(
            self._lib.jl_magat_nodes(ctypes.byref(self._magat), _stream(self._device)),
            "PyG node builder",
        )

    def _run_edges(self) -> None:
        check(
            self._lib.jl_magat_edges(ctypes.byref(self._magat), _stream(self._device)),
            "PyG edge builder",
        )

    # Narrowed views need the edge count on the host (bind.cpp:179-186).
    @property
    def pyg_edge_index(self) -> torch.Tensor:
        num_edges = int(self.t_pyg_num_edges.cpu().item())
        return self.t_pyg_edge_index_storage.narrow(1, 0, num_edges)

    @property
    def pyg_edge_attr(self) -> torch.Tensor:
        num_edges = int(self.t_pyg_num_edges.cpu().item())
        return self.t_pyg_edge_attr_storage.narrow(0, 0, num_edges)

    pyg_x = property(lambda self: self.t_pyg_x)
    pyg_pos = property(lambda self: self.t_pyg_pos)
    pyg_edge_index_storage = property(lambda self: self.t_pyg_edge_index_storage)
    pyg_edge_attr_storage = property(lambda self: self.t_pyg_edge_attr_storage)
    pyg_batch = property(lambda self: self.t_pyg_batch)
    pyg_ptr = property(lambda self: self.t_pyg_ptr)
    pyg_num_edges = property(lambda self: self.t_pyg_num_edges)


def _check_grids_strict(grids, W: int, H: int, *, long_messages: bool) -> None:
    if long_messages:  # MapfGPTObservationBuilder (mapf_gpt_builder.cpp:24-32)
        _require(isinstance(grids, torch.Tensor) and grids.is_cuda, "grids must be on a CUDA device")
        _require(grids.dtype == torch.int32, "grids must use int32 dtype")
        _require(grids.is_contiguous(), "grids must be contiguous")
        _require(
            grids.dim() == 3 and grids.size(1) == W and grids.size(2) == H,
            f"grids shape must be [n_envs, {W}, {H}]",
        )
    else:  # GridWorldSimulator (grid_world_simulator.cpp:181-188)
        _require(isinstance(grids, torch.Tensor) and grids.is_cuda, "grids must be CUDA")
        _require(grids.dtype == torch.int32, "grids must be int32")
        _require(grids.is_contiguous(), "grids must be contiguous")
        _require(
            grids.dim() == 3 and grids.size(1) == W and grids.size(2) == H,
            f"grids must have shape [n_envs, {W}, {H}]",
        )


class _Base:
    _MAP_W = 128
    _MAP_H = 128

    def _encode(self, grids: torch.Tensor) -> None:
        E = int(grids.shape[0])
        self.t_grid_compressed = torch.zeros(
            (E, self._MAP_W * self._MAP_H // 32), dtype=torch.int32, device=grids.device
        )
        check(
            self._lib.jl_encode_map(
                grids.data_ptr(),
                self.t_grid_compressed.data_ptr(),
                E,
                self._MAP_W,
                self._MAP_H,
                _stream(grids.device),
            ),
            "map encoding",
        )


# ---------------------------------------------------------------------------
# MapfGPTObservationBuilder (mapf_gpt_builder.h:24-51, bind.cpp:98-116)
# ---------------------------------------------------------------------------
class MapfGPTObservationBuilder(_Base):
    def __init__(self, grids, n_agents):
        W, H = self._MAP_W, self._MAP_H
        _check_grids_strict(grids, W, H, long_messages=True)
        n_agents = int(n_agents)
        _require(n_agents > 0, "n_agents must be positive")
        E = int(grids.size(0))
        _require(E > 0, "grids must contain at least one environment")
        self._lib = load_library()
        self.n_envs, self.n_agents = E, n_agents
        device = grids.device
        self._device = device
        N = E * n_agents
        with torch.cuda.device(device):
            self._encode(grids)
            self.t_state_packed = torch.zeros((N, 8), dtype=torch.int16, device=device)
            self.t_histories = torch.full((N, 5), 5, dtype=torch.int16, device=device)
            self.t_labels = torch.zeros((N,), dtype=torch.int64, device=device)
            self.t_tokens = torch.full((N, 256), 66, dtype=torch.int32, device=device)
            self.t_active_mask = torch.zeros((N,), dtype=torch.bool, device=device)
            self.t_cost_to_go = torch.full((E, n_agents, W, H), -1, dtype=torch.int16, device=device)
            self.t_agent_at_cell = torch.full((E, W, H), -1, dtype=torch.int32, device=device)
            self.t_goal_cache = torch.full((N, 2), -1, dtype=torch.int16, device=device)
            self.t_diagnostics = torch.zeros((4,), dtype=torch.int32, device=device)
            self.t_pyg_ptr = torch.arange(E + 1, dtype=torch.int64, device=device) * n_agents
            # build-private workspaces: per-agent greedy mask + diagnostic flags, and
            # the distance fields in 8x8 tiles with a one-tile border of unreachable
            # cells (the token pass reads its windows there); -1 is unreachable
            self._agent_info = torch.zeros((N,), dtype=torch.int32, device=device)
            self._cost_tiles = torch.full(
                (E, n_agents, tiled_field_cells(W, H)), -1, dtype=torch.int16, device=device
            )
            # single-launch builds: number of the last launch whose diagnostics
            # were cleared (uint64) and workgroup arrival counters; zero at
            # construction
            self._build_scratch = torch.zeros(
                (BUILD_SCRATCH_WORDS,), dtype=torch.int32, device=device
            )
        self._desc = MapfGPTDesc(
            n_envs=E,
            n_agents=n_agents,
            map_w=W,
            map_h=H,
            grid_bits=_ptr(self.t_grid_compressed),
            state_packed=_ptr(self.t_state_packed),
            histories=_ptr(self.t_histories),
            labels=_ptr(self.t_labels),
            cost_to_go=_ptr(self.t_cost_to_go),
            agent_at_cell=_ptr(self.t_agent_at_cell),
            goal_cache=_ptr(self.t_goal_cache),
            tokens=_ptr(self.t_tokens),
            active_mask=_ptr(self.t_active_mask),
            diagnostics=_ptr(self.t_diagnostics),
            agent_info=_ptr(self._agent_info),
            cost_tiles=_ptr(self._cost_tiles),
            build_scratch=_ptr(self._build_scratch),
        )
        self._desc_ref = ctypes.byref(self._desc)
        # stream of the last build: single-launch builds number themselves on
        # the device and must run one after another
        self._build_stream = None
        self._build_raw = None  # raw handle of _build_stream
        self._state_shape = torch.Size((self.n_envs, self.n_agents))

    def _order_builds(self) -> None:
        """Orders this build after the previous one when they are issued from
        different streams (single-launch builds derive their launch number
        from arrival counters that assume builds do not overlap).  Builds
        captured into a graph are ordered by the capture itself."""
        raw = _stream(self._device)
        if raw == self._build_raw:
            return  # the stream of the previous build: ordered already
        if torch.cuda.is_current_stream_capturing():
            return
        cur = torch.cuda.current_stream(self._device)
        last = self._build_stream
        if last is not None and last != cur:
            cur.wait_stream(last)
        self._build_stream = cur
        self._build_raw = raw

    def build_tokens(self, raw_rows: torch.Tensor) -> None:
        """mapf_gpt_builder.cpp:89-114."""
        _require(raw_rows.is_cuda, "raw_rows must be on a CUDA device")
        _require(raw_rows.dtype == torch.int16, "raw_rows must use int16 dtype")
        _require(raw_rows.dim() == 2, "raw_rows must be a 2D tensor")
        _require(raw_rows.size(1) == 13, "raw_rows feature dimension must be 13")
        _require(
            raw_rows.size(0) == self.n_envs * self.n_agents,
            "raw_rows row count must equal n_envs * n_agents",
        )
        _require(raw_rows.is_contiguous(), "raw_rows must be contiguous")
        _require(
            raw_rows.device == self._device,
            "raw_rows and builder tensors must use the same CUDA device",
        )
        self._order_builds()
        check(
            self._lib.jl_mapfgpt_build_rows(self._desc_ref, raw_rows.data_ptr(), _stream(self._device)),
            "MAPF-GPT cost-to-go generation",
        )

    @property
    def single_launch(self) -> bool:
        """True when a build runs as one launch (unpack, field refreshes and
        tokens of an env in one workgroup), eager or captured into a graph:
        maps of at most 4096 cells and at most 1024 agents per env.  No
        counterpart in the reference."""
        return bool(self._lib.jl_mapfgpt_single_launch(self._desc_ref))

    @property
    def single_launch_waits_given_up(self) -> int:
        """Workgroups of single-launch builds whose wait for their launch's
        cleared diagnostics reached its bound (the counts they added may have
        been cleared by that launch or not): 0 on a healthy builder.  Reads
        device memory (synchronises the builder's device); sticky until
        ``clear_single_launch_waits``.  No counterpart in the reference."""
        if self._build_scratch is None:
            return 0
        return int(self._build_scratch[GAVE_UP_WORD].item())

    def clear_single_launch_waits(self) -> None:
        """Resets the count read by ``single_launch_waits_given_up``."""
        if self._build_scratch is not None:
            self._build_scratch[GAVE_UP_WORD].zero_()

    def _check_state(self, t: torch.Tensor, name: str) -> None:
        if (t.dtype is torch.int16 and t.shape == self._state_shape and t.device == self._device
                and t.is_contiguous()):
            return  # valid: the checks below name the first failing condition otherwise
        _require(t.is_cuda, f"{name} must be on a CUDA device")
        _require(t.dtype == torch.int16, f"{name} must use int16 dtype")
        _require(
            t.dim() == 2 and t.size(0) == self.n_envs and t.size(1) == self.n_agents,
            f"{name} shape must be [n_envs, n_agents]",
        )
        _require(t.is_contiguous(), f"{name} must be contiguous")
        _require(t.device == self._device, f"{name} must use the builder CUDA device")

    def build_tokens_from_state(self, cur_x, cur_y, goal_x, goal_y) -> None:
        """mapf_gpt_builder.cpp:140-167."""
        for t, name in ((cur_x, "cur_x"), (cur_y, "cur_y"), (goal_x, "goal_x"), (goal_y, "goal_y")):
            self._check_state(t, name)
        self._order_builds()
        check(
            self._lib.jl_mapfgpt_build_state(
                self._desc_ref,
                cur_x.data_ptr(),
                cur_y.data_ptr(),
                goal_x.data_ptr(),
                goal_y.data_ptr(),
                _stream(self._device),
            ),
            "MAPF-GPT resident token generation",
        )

    def refresh_distances(self, cur_x, cur_y, goal_x, goal_y) -> None:
        """Goal-cache refresh and BFS of changed goals, no tokens
        (mapf_gpt_builder.cpp:200-212 of rebuttal/online-rl/native/src/cuda_backend)."""
        for t, name in ((cur_x, "cur_x"), (cur_y, "cur_y"), (goal_x, "goal_x"), (goal_y, "goal_y")):
            self._check_state(t, name)
        check(
            self._lib.jl_mapfgpt_refresh_state(
                self._desc_ref, cur_x.data_ptr(), cur_y.data_ptr(), goal_x.data_ptr(), goal_y.data_ptr(),
                _stream(self._device),
            ),
            "MAPF-GPT distance refresh",
        )

    def append_actions(self, actions: torch.Tensor) -> None:
        """mapf_gpt_builder.cpp:170-192."""
        if not (actions.dtype is torch.uint8 and actions.shape == self._state_shape
                and actions.device == self._device and actions.is_contiguous()):
            self._check_actions(actions)
        check(
            self._lib.jl_mapfgpt_append_actions(self._desc_ref, actions.data_ptr(), _stream(self._device)),
            "MAPF-GPT action-history update",
        )

    def _check_actions(self, actions: torch.Tensor) -> None:
        _require(actions.is_cuda, "actions must be on a CUDA device")
        _require(actions.dtype == torch.uint8, "actions must use uint8 dtype")
        _require(
            actions.dim() == 2 and actions.size(0) == self.n_envs and actions.size(1) == self.n_agents,
            "actions shape must be [n_envs, n_agents]",
        )
        _require(actions.is_contiguous(), "actions must be contiguous")
        _require(actions.device == self._device, "actions must use the builder CUDA device")

    def reset_histories(self) -> None:
        check(
            self._lib.jl_mapfgpt_reset_histories(self._desc_ref, _stream(self._device)),
            "MAPF-GPT history reset",
        )

    tokens = property(lambda self: self.t_tokens)
    active_mask = property(lambda self: self.t_active_mask)
    labels = property(lambda self: self.t_labels)
    @property
    def cost_to_go(self) -> torch.Tensor:
        """Exact BFS distances [E, A, W, H] (-1 = unreachable), filled from the
        tiled fields on every read, on the current stream, so that builds
        replayed from captured graphs are seen as well (the reference writes
        them on every refresh, mapf_gpt_cuda.cu:318-325).  The tensor is the
        same object on every read, but its contents are a snapshot of the
        builds before that read: builds write only the private tiled copy,
        so a caller that keeps the tensor must read ``builder.cost_to_go``
        again after a build to see it."""
        check(
            self._lib.jl_mapfgpt_cost_to_go(self._desc_ref, _stream(self._device)),
            "MAPF-GPT cost-to-go copy",
        )
        return self.t_cost_to_go
    state_packed = property(lambda self: self.t_state_packed)
    histories = property(lambda self: self.t_histories)
    diagnostics = property(lambda self: self.t_diagnostics)
    pyg_ptr = property(lambda self: self.t_pyg_ptr)
    goal_cache = property(lambda self: self.t_goal_cache)

    @property
    def agent_at_cell(self) -> torch.Tensor:
        """Cell -> agent id map of the last build (-1 empty), filled on read:
        like ``cost_to_go``, a snapshot that a kept tensor does not follow
        into later builds."""
        check(
            self._lib.jl_mapfgpt_agent_at_cell(self._desc_ref, _stream(self._device)),
            "MAPF-GPT agent identity grid",
        )
        return self.t_agent_at_cell

    @property
    def memory_tensors(self) -> dict:
        """The builder's tensors (bind.cpp:98-116).  ``cost_to_go`` and
        ``agent_at_cell`` are filled when this dict is read: snapshots of the
        builds so far, to be read again through the attributes after a
        later build."""
        return {
            "grid_compressed": self.t_grid_compressed,
            "state_packed": self.t_state_packed,
            "histories": self.t_histories,
            "labels": self.t_labels,
            "tokens": self.t_tokens,
            "active_mask": self.t_active_mask,
            "cost_to_go": self.cost_to_go,
            "agent_at_cell": self.agent_at_cell,
            "goal_cache": self.t_goal_cache,
            "diagnostics": self.t_diagnostics,
            "pyg_ptr": self.t_pyg_ptr,
        }


# ---------------------------------------------------------------------------
# GridWorldSimulator (grid_world_simulator.h:9-107, bind.cpp:118-200)
# ---------------------------------------------------------------------------
class GridWorldSimulator(_Base, _PygModeMixin, _PygStorage):
    def __init__(
        self,
        grids,
        n_agents,
        num_features,
        pool_capacity,
        seed,
        task_mode="lifelong",
        max_episode_steps=256,
    ):
        W, H = self._MAP_W, self._MAP_H
        _check_grids_strict(grids, W, H, long_messages=False)
        mode = _parse_task_mode(task_mode)
        max_episode_steps = int(max_episode_steps)
        _require(max_episode_steps > 0, "max_episode_steps must be positive")
        n_agents = int(n_agents)
        _require(n_agents > 0, "n_agents must be positive")
        self._lib = load_library()
        E = int(grids.size(0))
        self.n_envs, self.n_agents = E, n_agents
        self._task_mode = mode
        self._max_episode_steps = max_episode_steps
        self.current_step = 0
        self._builder_mode = "auto"
        self._gather_impl = "auto"
        device = grids.device
        self._device = device
        N = E * n_agents
        i16 = dict(dtype=torch.int16, device=device)
        i32 = dict(dtype=torch.int32, device=device)
        u8 = dict(dtype=torch.uint8, device=device)
        with torch.cuda.device(device):
            self._encode(grids)
            self.t_max_free_cell_count = torch.zeros((1,), **i32)
            # free cells of env e live at [e*W*H, e*W*H + count) (deterministic layout)
            self.t_free_cell_list = torch.zeros((max(int(pool_capacity), E * W * H),), **i32)
            self.t_pool_ptr = torch.zeros((1,), **i32)
            self.t_offsets = torch.full((E,), -1, **i32)
            self.t_counts = torch.zeros((E,), **i32)
            self.t_real_map_extents = torch.empty((E, 2), **i32)
            self.t_real_map_extents[:, 0] = W
            self.t_real_map_extents[:, 1] = H
            self.t_grid_ocp = torch.zeros((E, W * H // 32), **i32)
            self.t_cur_x = torch.zeros((E, n_agents), **i16)
            self.t_cur_y = torch.zeros((E, n_agents), **i16)
            self.t_goals_x = torch.zeros((E, n_agents), **i16)
            self.t_goals_y = torch.zeros((E, n_agents), **i16)
            self.t_agents_obs = torch.zeros((N, int(num_features), 2 * RADIUS + 1), **i16)
            self.t_rewards = torch.zeros((E, n_agents), dtype=torch.float32, device=device)
            self.t_actions = torch.zeros((E, n_agents), **u8)
            self.t_goal_changed_flags = torch.zeros((E, n_agents), **u8)
            self.t_arrived = torch.zeros((E, n_agents), **u8)
            self.t_terminated = torch.zeros((E,), **u8)
            self.t_truncated = torch.zeros((E,), **u8)
            self.t_step_counts = torch.zeros((E,), **i32)
            self.t_outcomes = torch.zeros((E, n_agents), **u8)
            self.t_energy_maps = torch.zeros((E, n_agents, W, H), **u8)
            self.t_state_packed = torch.zeros((N, 8), **i16)
            self._alloc_pyg(E, n_agents, device)
            self.t_goal_changed_prefix = torch.zeros((N,), dtype=torch.int64, device=device)
            self.t_changed_state_packed = torch.zeros((N, 8), **i16)
            self.t_goal_changed_count = torch.zeros((1,), dtype=torch.int64, device=device)
            self.t_rng_states = torch.zeros((E * max(n_agents, 32),), dtype=torch.int64, device=device)
        # deterministic lifelong goals (set_goal_candidates); unset = generator draws
        self.t_goal_candidates = None
        self.t_candidate_cells = None
        self.t_candidate_counts = None
        self.t_goal_cursors = None
        self._sim = self._make_sim_desc()
        self._sim_ref = ctypes.byref(self._sim)
        self._magat = self._magat_desc(self.t_state_packed, self.t_energy_maps)
        self.init_rng(seed)

    def _make_sim_desc(self) -> SimDesc:
        return SimDesc(
            n_envs=self.n_envs,
            n_agents=self.n_agents,
            map_w=self._MAP_W,
            map_h=self._MAP_H,
            task_mode=self._task_mode,
            max_episode_steps=self._max_episode_steps,
            grid_bits=_ptr(self.t_grid_compressed),
            grid_ocp=_ptr(self.t_grid_ocp),
            cur_x=_ptr(self.t_cur_x),
            cur_y=_ptr(self.t_cur_y),
            goal_x=_ptr(self.t_goals_x),
            goal_y=_ptr(self.t_goals_y),
            actions=_ptr(self.t_actions),
            arrived=_ptr(self.t_arrived),
            goal_changed=_ptr(self.t_goal_changed_flags),
            rewards=_ptr(self.t_rewards),
            terminated=_ptr(self.t_terminated),
            truncated=_ptr(self.t_truncated),
            step_counts=_ptr(self.t_step_counts),
            state_packed=_ptr(self.t_state_packed),
            outcomes=_ptr(self.t_outcomes),
            free_cells=_ptr(self.t_free_cell_list),
            env_offsets=_ptr(self.t_offsets),
            env_counts=_ptr(self.t_counts),
            rng_state=_ptr(self.t_rng_states),
            goal_candidates=_ptr(self.t_goal_candidates),
            candidate_cells=_ptr(self.t_candidate_cells),
            candidate_counts=_ptr(self.t_candidate_counts),
            goal_cursors=_ptr(self.t_goal_cursors),
            candidate_length=0 if self.t_goal_candidates is None else int(self.t_goal_candidates.size(2)),
            candidate_stride=0 if self.t_candidate_cells is None else int(self.t_candidate_cells.size(1)),
        )

    def set_goal_candidates(self, candidates: torch.Tensor, cells: torch.Tensor, counts: torch.Tensor) -> None:
        """Deterministic lifelong goals (grid_world_simulator.cpp:901-918 of
        rebuttal/online-rl/native/src/cuda_backend): agent i on its goal takes
        the first cell of its env's list ``cells[e, :counts[e]]``, starting at
        ``candidates[e, i, cursor % K]``, that is neither its own cell nor a
        goal held by another agent; agents are served in id order, so the
        result is the one the CPU twin (rebuttal/online-il/tasks.py:51-65)
        computes.  Resets ``goal_cursors`` to zero."""
        dev = self._device
        _require(candidates.is_cuda and cells.is_cuda and counts.is_cuda, "goal candidates must be CUDA")
        _require(candidates.device == dev and cells.device == dev and counts.device == dev,
                 "goal source device mismatch")
        _require(candidates.dtype == torch.int32 and cells.dtype == torch.int16 and counts.dtype == torch.int32,
                 "goal source dtype mismatch")
        _require(candidates.dim() == 3 and candidates.size(0) == self.n_envs
                 and candidates.size(1) == self.n_agents and candidates.size(2) > 0, "candidates must be [N,A,K]")
        _require(cells.dim() == 3 and cells.size(0) == self.n_envs and cells.size(2) == 2, "cells must be [N,F,2]")
        _require(counts.numel() == self.n_envs and int(counts.min().item()) > self.n_agents
                 and int(counts.max().item()) <= cells.size(1), "invalid free-cell counts")
        with torch.cuda.device(dev):
            self.t_goal_candidates = candidates.contiguous()
            self.t_candidate_cells = cells.contiguous()
            self.t_candidate_counts = counts.contiguous()
            self.t_goal_cursors = torch.zeros((self.n_envs, self.n_agents), dtype=torch.int32, device=dev)
        self._sim = self._make_sim_desc()
        self._sim_ref = ctypes.byref(self._sim)

    @property
    def goal_cursors(self):
        """Goals taken per agent since set_goal_candidates (bind.cpp:135 of the online-rl fork)."""
        return self.t_goal_cursors

    # -- lifecycle ---------------------------------------------------------
    def init_rng(self, seed) -> None:
        """Seed the per-agent goal-sampling generators (grid_world_simulator.cpp:628-637)."""
        check(
            self._lib.jl_seed_rng(
                self.t_rng_states.data_ptr(),
                int(self.t_rng_states.numel()),
                int(seed) & 0xFFFFFFFFFFFFFFFF,
                _stream(self._device),
            ),
            "setup_rng",
        )

    def run_initialization(self) -> None:
        """Free-cell lists and random distinct starts/goals (grid_world_simulator.cpp:646-676)."""
        with torch.cuda.device(self._device):
            self.current_step = 0
            for t in (
                self.t_arrived,
                self.t_terminated,
                self.t_truncated,
                self.t_step_counts,
                self.t_goal_changed_flags,
                self.t_actions,
                self.t_pool_ptr,
            ):
                t.zero_()
            check(
                self._lib.jl_lifelong_init(
                    self._sim_ref,
                    self.t_real_map_extents.data_ptr(),
                    self.t_free_cell_list.data_ptr(),
                    self.t_offsets.data_ptr(),
                    self.t_counts.data_ptr(),
                    _stream(self._device),
                ),
                "lifelong initialisation",
            )
            self.t_max_free_cell_count.copy_(self.t_counts.max().reshape(1))
            # every agent takes two distinct cells; with fewer the reference's
            # slot search (utils_cuda.h:39-61) never ends, here it raises
            fewest = int(self.t_counts.min().item())
            _require(
                fewest >= 2 * self.n_agents,
                f"run_initialization needs 2 * n_agents = {2 * self.n_agents} free cells inside every env's "
                f"real extent (distinct starts and goals); an env has {fewest}",
            )

    def update_actions(self, new_actions: torch.Tensor) -> None:
        """grid_world_simulator.cpp:678-688."""
        if not (new_actions.dtype is torch.uint8 and new_actions.shape == self.t_actions.shape
                and new_actions.device == self._device and new_actions.is_contiguous()):
            _require(new_actions.dtype == torch.uint8, "new_actions must be uint8")
            _require(new_actions.is_cuda, "new_actions must be CUDA")
            _require(new_actions.shape == self.t_actions.shape, "new_actions shape mismatch")
            _require(new_actions.is_contiguous(), "new_actions must be contiguous")
            _require(
                new_actions.device == self._device,
                "new_actions and simulator tensors must use the same CUDA device",
            )
        check(
            self._lib.jl_update_actions(self._sim_ref, _ptr(new_actions), _stream(self._device)),
            "update_actions",
        )

    def step_sim_only(self) -> None:
        """grid_world_simulator.cpp:694-705."""
        self.current_step += 1
        check(self._lib.jl_step(self._sim_ref, _stream(self._device)), "Step kernel")

    def step_compact_only(self) -> None:
        self.step_sim_only()

    def update_derived_state(self) -> None:
        """Energy fields of changed goals (grid_world_simulator.cpp:707-753), no host sync."""
        if self.current_step != 1:
            # the changed-row buffer is cleared, then packed; the fields of
            # the changed goals are refreshed
            check(
                self._lib.jl_goal_changed_refresh(
                    self._sim_ref,
                    self.t_energy_maps.data_ptr(),
                    self.t_goal_changed_prefix.data_ptr(),
                    self.t_goal_changed_count.data_ptr(),
                    self.t_changed_state_packed.data_ptr(),
                    _stream(self._device),
                ),
                "Incremental energy map kernel",
            )
            return
        check(
            self._lib.jl_goal_changed_scan(
                self._sim_ref,
                self.t_goal_changed_prefix.data_ptr(),
                self.t_goal_changed_count.data_ptr(),
                None,
                _stream(self._device),
            ),
            "Goal-changed scan",
        )
        check(
            self._lib.jl_energy_maps_flagged(
                self._sim_ref,
                self.t_energy_maps.data_ptr(),
                1,
                self.t_goal_changed_prefix.data_ptr(),
                self.t_changed_state_packed.data_ptr(),
                _stream(self._device),
            ),
            "Stateful energy map kernel",
        )

    def build_magat_plus_nodes(self) -> None:
        self._run_nodes()

    def finalize_magat_plus_graph(self) -> None:
        self._run_edges()

    def build_magat_plus_inputs(self) -> None:
        self._run_nodes()
        self._run_edges()

    def materialize_pyg_inputs(self) -> None:
        self.build_magat_plus_inputs()

    def step_and_build_pyg(self) -> None:
        self.step_sim_only()
        self.update_derived_state()
        self.materialize_pyg_inputs()

    def step(self) -> None:
        self.step_and_build_pyg()

    def set_real_map_extents(self, real_map_extents: torch.Tensor) -> None:
        """grid_world_simulator.cpp:471-492."""
        _require(real_map_extents.dtype == torch.int32, "real_map_extents must be int32")
        _require(real_map_extents.dim() == 2, "real_map_extents must be 2D [n_envs, 2]")
        _require(real_map_extents.size(0) == self.n_envs, "real_map_extents must have one row per env")
        _require(real_map_extents.size(1) == 2, "real_map_extents must have shape [n_envs, 2]")
        ext = real_map_extents.contiguous().to(device=self._device, dtype=torch.int32)
        host = ext.cpu()
        W, H = self._MAP_W, self._MAP_H
        for env_id in range(self.n_envs):
            w, h = int(host[env_id, 0]), int(host[env_id, 1])
            _require(0 < w <= W, f"real_map_extents[:, 0] must be in [1, {W}]")
            _require(0 < h <= H, f"real_map_extents[:, 1] must be in [1, {H}]")
        self.t_real_map_extents = ext.clone()

    def load_state(self, positions, goals, arrived, step_counts) -> None:
        """grid_world_simulator.cpp:502-591."""
        E, A = self.n_envs, self.n_agents
        for t, name, dtype, dname, shape, sname in (
            (positions, "positions", torch.int16, "int16", (E, A, 2), "[n_envs, n_agents, 2]"),
            (goals, "goals", torch.int16, "int16", (E, A, 2), "[n_envs, n_agents, 2]"),
            (arrived, "arrived", torch.uint8, "uint8", (E, A), "[n_envs, n_agents]"),
            (step_counts, "step_counts", torch.int32, "int32", (E,), "[n_envs]"),
        ):
            _require(t.is_cuda, f"{name} must be CUDA")
            _require(t.dtype == dtype, f"{name} must be {dname}")
            _require(tuple(t.shape) == shape, f"{name} must have shape {sname}")
            _require(t.is_contiguous(), f"{name} must be contiguous")
            _require(
                t.device == self._device,
                f"{name} and simulator tensors must use the same CUDA device",
            )
        W, H = self._MAP_W, self._MAP_H
        with torch.cuda.device(self._device):
            px, py = positions[..., 0], positions[..., 1]
            gx, gy = goals[..., 0], goals[..., 1]
            oob = (
                bool((px < 0).any()) or bool((px >= W).any())
                or bool((py < 0).any()) or bool((py >= H).any())
                or bool((gx < 0).any()) or bool((gx >= W).any())
                or bool((gy < 0).any()) or bool((gy >= H).any())
            )
            _require(not oob, "position and goal coordinates must be within map bounds")
            _require(not bool((arrived > 1).any()), "arrived values must be 0 or 1")
            on_goal = (positions == goals).all(dim=2)
            _require(
                not bool((arrived.bool() & ~on_goal).any()),
                "arrived agents must be at their goals",
            )
            _require(
                not bool((step_counts < 0).any())
                and not bool((step_counts > self._max_episode_steps).any()),
                "step_counts must be in [0, max_episode_steps]",
            )
            self.current_step = 0
            check(
                self._lib.jl_load_state(
                    self._sim_ref,
                    positions.data_ptr(),
                    goals.data_ptr(),
                    arrived.data_ptr(),
                    step_counts.data_ptr(),
                    _stream(self._device),
                ),
                "load_state kernel",
            )

    def decode_to_uint8(self) -> torch.Tensor:
        """Legacy observation decode (grid_world_simulator.cpp:861-882)."""
        n_batch = self.n_envs * self.n_agents
        d = 2 * RADIUS + 1
        with torch.cuda.device(self._device):
            out = torch.empty((n_batch, 2, d, d), dtype=torch.uint8, device=self._device)
            check(
                self._lib.jl_decode_to_uint8(
                    self.t_agents_obs.data_ptr(), out.data_ptr(), n_batch, d, _stream(self._device)
                ),
                "Decode kernel",
            )
        return out

    # -- properties --------------------------------------------------------
    @property
    def task_mode(self) -> str:
        return _TASK_NAMES[self._task_mode]

    @property
    def max_episode_steps(self) -> int:
        return self._max_episode_steps

    agents_obs = property(lambda self: self.t_agents_obs)
    rewards = property(lambda self: self.t_rewards)
    actions = property(lambda self: self.t_actions)
    cur_x = property(lambda self: self.t_cur_x)
    cur_y = property(lambda self: self.t_cur_y)
    goal_x = property(lambda self: self.t_goals_x)
    goal_y = property(lambda self: self.t_goals_y)
    grid_ocp = property(lambda self: self.t_grid_ocp)
    state_packed = property(lambda self: self.t_state_packed)
    counts = property(lambda self: self.t_counts)
    energy_maps = property(lambda self: self.t_energy_maps)
    goal_changed_flags = property(lambda self: self.t_goal_changed_flags)
    arrived = property(lambda self: self.t_arrived)
    terminated = property(lambda self: self.t_terminated)
    truncated = property(lambda self: self.t_truncated)
    step_counts = property(lambda self: self.t_step_counts)
    goal_changed_prefix = property(lambda self: self.t_goal_changed_prefix)
    changed_state_packed = property(lambda self: self.t_changed_state_packed)
    goal_changed_count = property(lambda self: self.t_goal_changed_count)
    # Conflict outcome of the last step per agent: 0 none, 1 wall, 2 vertex,
    # 3 swap, 4 chain (the categories of transition_adapters.py:361-455).
    outcomes = property(lambda self: self.t_outcomes)

    @property
    def memory_tensors(self) -> dict:
        return {
            "grid_compressed": self.t_grid_compressed,
            "free_cell_list": self.t_free_cell_list,
            "pool_ptr": self.t_pool_ptr,
            "offsets": self.t_offsets,
            "counts": self.t_counts,
            "grid_ocp": self.t_grid_ocp,
            "real_map_extents": self.t_real_map_extents,
            "cur_x": self.t_cur_x,
            "cur_y": self.t_cur_y,
            "goal_x": self.t_goals_x,
            "goal_y": self.t_goals_y,
            "agents_obs": self.t_agents_obs,
            "rewards": self.t_rewards,
            "actions": self.t_actions,
            "rng_states": self.t_rng_states,
            "max_free_cell_count": self.t_max_free_cell_count,
            "goal_changed_flags": self.t_goal_changed_flags,
            "arrived": self.t_arrived,
            "terminated": self.t_terminated,
            "truncated": self.t_truncated,
            "step_counts": self.t_step_counts,
            "goal_changed_prefix": self.t_goal_changed_prefix,
            "changed_state_packed": self.t_changed_state_packed,
            "goal_changed_count": self.t_goal_changed_count,
            "energy_maps": self.t_energy_maps,
            "state_packed": self.t_state_packed,
            "pyg_x": self.t_pyg_x,
            "pyg_pos": self.t_pyg_pos,
            "pyg_edge_index": self.t_pyg_edge_index,
            "pyg_edge_attr": self.t_pyg_edge_attr,
            "pyg_batch": self.t_pyg_batch,
            "pyg_ptr": self.t_pyg_ptr,
            "pyg_num_edges": self.t_pyg_num_edges,
            "edge_counts": self.t_edge_counts,
            "pyg_edge_index_storage": self.t_pyg_edge_index_storage,
            "pyg_edge_attr_storage": self.t_pyg_edge_attr_storage,
            "pyg_edge_prefix": self.t_pyg_edge_prefix,
            "scan_temp_storage": self.t_scan_temp_storage,
        }

    # -- debug printers (print_tensor.cpp) ----------------------------------
    def _print(self, name: str) -> None:
        print(name, getattr(self, name).cpu())

    def print_t_grid_compressed(self): self._print("t_grid_compressed")
    def print_t_free_cell_list(self): self._print("t_free_cell_list")
    def print_t_pool_ptr(self): self._print("t_pool_ptr")
    def print_t_offsets(self): self._print("t_offsets")
    def print_t_counts(self): self._print("t_counts")
    def print_t_grid_ocp(self): self._print("t_grid_ocp")
    def print_t_cur_x(self): self._print("t_cur_x")
    def print_t_cur_y(self): self._print("t_cur_y")
    def print_t_goals_x(self): self._print("t_goals_x")
    def print_t_goals_y(self): self._print("t_goals_y")
    def print_t_agents_obs(self): self._print("t_agents_obs")
    def print_t_rewards(self): self._print("t_rewards")
    def print_t_actions(self): self._print("t_actions")
    def print_t_max_free_cell_count(self): self._print("t_max_free_cell_count")


# ---------------------------------------------------------------------------
# StatelessGridWorldSimulator (grid_world_simulator.h:109-144, bind.cpp:202-236)
# ---------------------------------------------------------------------------
class StatelessGridWorldSimulator(_Base, _PygModeMixin, _PygStorage):
    def __init__(self, grids, n_agents, num_features=3):
        W, H = self._MAP_W, self._MAP_H
        _require(
            isinstance(grids, torch.Tensor)
            and grids.dim() == 3 and grids.size(1) == W and grids.size(2) == H,
            f"grids must have shape [n_envs, {W}, {H}]",
        )
        _require(grids.is_cuda, "grids must be CUDA")
        _require(grids.dtype == torch.int32, "grids must be int32")
        _require(grids.is_contiguous(), "grids must be contiguous")
        n_agents = int(n_agents)
        _require(n_agents > 0, "n_agents must be positive")
        self._lib = load_library()
        E = int(grids.size(0))
        self.n_envs, self.n_agents = E, n_agents
        self._builder_mode = "auto"
        self._gather_impl = "auto"
        device = grids.device
        self._device = device
        N = E * n_agents
        with torch.cuda.device(device):
            self._encode(grids)
            self.t_grid_ocp = torch.zeros((E, W * H // 32), dtype=torch.int32, device=device)
            self.t_energy_maps = torch.zeros((E, n_agents, W, H), dtype=torch.uint8, device=device)
            self.t_goals_x = torch.zeros((E, n_agents), dtype=torch.int16, device=device)
            self.t_goals_y = torch.zeros((E, n_agents), dtype=torch.int16, device=device)
            self.t_state_packed = torch.zeros((N, 8), dtype=torch.int16, device=device)
            self._alloc_pyg(E, n_agents, device)
        self._magat = self._magat_desc(self.t_state_packed, self.t_energy_maps)

    def _check_states(self, states: torch.Tensor) -> None:
        _require(states.is_cuda, "states_tensor must be on CUDA device")
        _require(states.dtype == torch.int16, "states_tensor must be int16")
        _require(states.dim() == 2, "states_tensor must be 2D (N, 8)")
        _require(states.size(1) == 8, "states_tensor feature dimension must be 8")
        _require(states.is_contiguous(), "states_tensor must be contiguous")

    def refresh_compact_state_from_raw_batch(self, states_tensor: torch.Tensor) -> None:
        """grid_world_simulator.cpp:439-454."""
        self._check_states(states_tensor)
        _require(
            states_tensor.size(0) <= self.t_state_packed.size(0),
            "states_tensor length exceeds preallocated stateless capacity",
        )
        with torch.cuda.device(self._device):
            self.t_state_packed.fill_(-1)
            self.t_state_packed.narrow(0, 0, states_tensor.size(0)).copy_(states_tensor)
            self.t_grid_ocp.zero_()
            check(
                self._lib.jl_magat_occupancy(ctypes.byref(self._magat), _stream(self._device)),
                "occupancy refresh",
            )

    def materialize_pyg_inputs(self) -> None:
        self._run_nodes()
        self._run_edges()

    def update_derived_state(self, states_tensor: torch.Tensor, length: int) -> None:
        self.update_energy_maps(states_tensor, length)

    def build_magat_plus_nodes(self, states_tensor: torch.Tensor) -> None:
        self.refresh_compact_state_from_raw_batch(states_tensor)
        self._run_nodes()

    def finalize_magat_plus_graph(self) -> None:
        self._run_edges()

    def build_magat_plus_inputs(self, states_tensor: torch.Tensor) -> None:
        self.refresh_compact_state_from_raw_batch(states_tensor)
        self.materialize_pyg_inputs()

    def setup_imitation_obs(self, states_tensor: torch.Tensor) -> None:
        self.refresh_compact_state_from_raw_batch(states_tensor)
        self.materialize_pyg_inputs()

    def update_energy_maps(self, states_tensor: torch.Tensor, length: int) -> None:
        """energy_map.cu:255-272 over the first `length` rows."""
        self._check_states(states_tensor)
        length = int(length)
        _require(0 <= length <= states_tensor.size(0), "length exceeds states_tensor rows")
        check(
            self._lib.jl_energy_maps(
                self.t_grid_compressed.data_ptr(),
                self.t_energy_maps.data_ptr(),
                states_tensor.data_ptr(),
                length,
                self.n_envs,
                self.n_agents,
                self._MAP_W,
                self._MAP_H,
                0,
                _stream(self._device),
            ),
            "Energy map kernel",
        )

    grid_ocp = property(lambda self: self.t_grid_ocp)
    state_packed = property(lambda self: self.t_state_packed)
    energy_maps = property(lambda self: self.t_energy_maps)

    @property
    def memory_tensors(self) -> dict:
        return {
            "grid_compressed": self.t_grid_compressed,
            "grid_ocp": self.t_grid_ocp,
            "state_packed": self.t_state_packed,
            "goal_x": self.t_goals_x,
            "goal_y": self.t_goals_y,
            "energy_maps": self.t_energy_maps,
            "pyg_x": self.t_pyg_x,
            "pyg_pos": self.t_pyg_pos,
            "pyg_edge_index": self.t_pyg_edge_index,
            "pyg_edge_attr": self.t_pyg_edge_attr,
            "pyg_batch": self.t_pyg_batch,
            "pyg_ptr": self.t_pyg_ptr,
            "pyg_num_edges": self.t_pyg_num_edges,
            "edge_counts": self.t_edge_counts,
            "pyg_edge_index_storage": self.t_pyg_edge_index_storage,
            "pyg_edge_attr_storage": self.t_pyg_edge_attr_storage,
            "pyg_edge_prefix": self.t_pyg_edge_prefix,
            "scan_temp_storage": self.t_scan_temp_storage,
        }


# ---------------------------------------------------------------------------
# Map profiles
# ---------------------------------------------------------------------------
SUPPORTED_H = tuple(range(32, 257, 32))
MAX_MAP_W = 256
_PROFILES: dict = {}


def parse_profile(text: str) -> tuple[int, int]:
    """'WxH' -> (W, H), with the checks and messages of setup.py:9-40
    (format, integers, positive, H a multiple of 32), plus this build's
    limit of 256 on both sides (the LDS and the 16-bit coordinates the
    kernels hold)."""
    profile_text = text.strip().lower()
    if "x" not in profile_text:
        raise ValueError(
            f"MAPF_CUDA_MAP_PROFILE must look like '<width>x<height>', got {profile_text!r}"
        )
    w_text, h_text = profile_text.split("x", 1)
    try:
        w, h = int(w_text), int(h_text)
    except ValueError as exc:
        raise ValueError(
            f"MAPF_CUDA_MAP_PROFILE must contain integer width/height, got {profile_text!r}"
        ) from exc
    if w <= 0 or h <= 0:
        raise ValueError(f"MAPF_CUDA_MAP_PROFILE must be positive, got {profile_text!r}")
    if h % 32 != 0:
        raise ValueError(
            "MAPF_CUDA_MAP_PROFILE height must be a multiple of 32 so the "
            f"compressed column layout stays integral, got {profile_text!r}"
        )
    if w > MAX_MAP_W or h not in SUPPORTED_H:
        raise ValueError(
            f"unsupported map profile {w}x{h}: this build takes 1 <= W <= {MAX_MAP_W} and "
            f"H in {SUPPORTED_H}"
        )
    return w, h


# ---------------------------------------------------------------------------
# CostTracer (rebuttal/online-rl/native/src/cuda_backend/costtracer.cu:87-127,
# bound as module functions in bind.cpp:96-98 of that tree)
# ---------------------------------------------------------------------------
def _ct_check(t, dtype, n, device) -> None:
    _require(
        isinstance(t, torch.Tensor) and t.is_cuda and t.is_contiguous() and t.dtype == dtype
        and t.numel() == n and t.device == device,
        "CostTracer tensor shape/dtype/device mismatch",
    )


def _ct_pair(sim, builder) -> None:
    _require(
        builder.n_envs == sim.n_envs and builder.n_agents == sim.n_agents
        and builder._MAP_W == sim._MAP_W and builder._MAP_H == sim._MAP_H and builder._device == sim._device,
        "CostTracer simulator and builder must share envs, agents, map size and device",
    )


def costtracer_reward_goals(sim, builder, best, targets, cursor, rewards, reached) -> None:
    """Progress rewards, goal hits and the next goals of the streams
    (costtracer.cu:87-103)."""
    n = sim.n_envs * sim.n_agents
    dev = sim._device
    _ct_pair(sim, builder)
    _ct_check(best, torch.int32, n, dev)
    _ct_check(cursor, torch.int32, n, dev)
    _ct_check(rewards, torch.float32, n, dev)
    _ct_check(reached, torch.float32, n, dev)
    _require(
        targets.dim() == 4 and targets.size(0) == sim.n_envs and targets.size(1) == sim.n_agents
        and targets.size(2) > sim.max_episode_steps and targets.size(3) == 2,
        "goal stream must be [N,A,K>horizon,2]",
    )
    _ct_check(targets, torch.int16, targets.numel(), dev)
    check(
        sim._lib.jl_costtracer_reward_goals(
            sim._sim_ref, builder._desc_ref, best.data_ptr(), targets.data_ptr(), int(targets.size(2)),
            cursor.data_ptr(), rewards.data_ptr(), reached.data_ptr(), _stream(dev),
        ),
        "CostTracer reward",
    )


def costtracer_observe(sim, builder, best, output) -> None:
    """2 x 11 x 11 observation per agent (costtracer.cu:105-113)."""
    n = sim.n_envs * sim.n_agents
    dev = sim._device
    _ct_pair(sim, builder)
    _ct_check(best, torch.int32, n, dev)
    _ct_check(output, torch.float32, n * 242, dev)
    check(
        sim._lib.jl_costtracer_observe(sim._sim_ref, builder._desc_ref, best.data_ptr(), output.data_ptr(),
                                       _stream(dev)),
        "CostTracer observation",
    )


def costtracer_reset(sim, pos, goal, episodes, cursors, best, reserved, horizon) -> None:
    """Envs at the horizon start the next episode of the bank
    (costtracer.cu:115-127); ``reserved`` is unused, as there."""
    n = sim.n_envs * sim.n_agents
    dev = sim._device
    _require(
        pos.dim() == 4 and pos.size(1) == sim.n_envs and pos.size(2) == sim.n_agents and pos.size(3) == 2,
        "reset bank must be [episodes,N,A,2]",
    )
    _ct_check(pos, torch.int16, pos.numel(), dev)
    _ct_check(goal, torch.int16, pos.numel(), dev)
    _ct_check(episodes, torch.int32, sim.n_envs, dev)
    _ct_check(cursors, torch.int32, n, dev)
    _ct_check(best, torch.int32, n, dev)
    check(
        sim._lib.jl_costtracer_reset(
            sim._sim_ref, pos.data_ptr(), goal.data_ptr(), int(pos.size(0)), episodes.data_ptr(),
            cursors.data_ptr(), best.data_ptr(), int(horizon), _stream(dev),
        ),
        "CostTracer reset",
    )


def profile(w: int, h: int) -> types.SimpleNamespace:
    """Module-like namespace with COMPILED_MAP_W/H and the three classes for a WxH map."""
    key = (int(w), int(h))
    parse_profile(f"{key[0]}x{key[1]}")
    if key not in _PROFILES:
        attrs = {"_MAP_W": key[0], "_MAP_H": key[1]}
        _PROFILES[key] = types.SimpleNamespace(
            COMPILED_MAP_W=key[0],
            COMPILED_MAP_H=key[1],
            MapfGPTObservationBuilder=type("MapfGPTObservationBuilder", (MapfGPTObservationBuilder,), attrs),
            GridWorldSimulator=type("GridWorldSimulator", (GridWorldSimulator,), attrs),
            StatelessGridWorldSimulator=type(
                "StatelessGridWorldSimulator", (StatelessGridWorldSimulator,), attrs
            ),
            costtracer_reward_goals=costtracer_reward_goals,
            costtracer_observe=costtracer_observe,
            costtracer_reset=costtracer_reset,
        )
    return _PROFILES[key]


def default_profile() -> types.SimpleNamespace:
    """The profile MAPF_CUDA_MAP_PROFILE names; 128x128 when it is unset or
    empty (setup.py:10-12)."""
    text = os.environ.get("MAPF_CUDA_MAP_PROFILE", "").strip()
    return profile(*parse_profile(text or "128x128"))
