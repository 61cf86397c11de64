"""HIP-graph capture of the resident loops.

The reference launches every kernel of a step from the host each step
(minimal_p0_mapf_gpt_resident_runner.py:256-281 for the MAPF-GPT loop,
fixed_magat_plus_runtime.py:53-115 with GridWorldSimulator::step_and_build_pyg,
grid_world_simulator.cpp:694-785, for the MAGAT loop).  Here one step of
either loop is captured once into a HIP graph (torch.cuda.CUDAGraph on ROCm)
and replayed: every launch of the step goes to the current stream, none
allocates, synchronises with the host or records a memset node (buffers are
cleared by fill kernels), so the captured step equals the eager one.

The step's actions: ``replay(actions)`` points the captured kernels that
read them (the history append and the action copy) at the given tensor
before launching (jl_graph_retarget_actions, host-side only), so each
replay reads that step's actions where they lie; ``replay()`` reads
``actions``, a tensor owned by the graph object that the caller may fill.
A tensor passed to ``replay`` is held until the next ``replay`` and must not
be written before that replay's work has run on the stream.  Objects
captured in a graph must stay alive and must not be re-created while the
graph is in use.  The host-side step counter of the simulator is advanced by
``replay`` as an eager step would.
"""
from __future__ import annotations

import ctypes

import torch

from ._abi import check, load_library


class _CapturedStep:
    def __init__(self, device: torch.device, body, actions: torch.Tensor, action_nodes: int) -> None:
        self._device = device
        self.actions = actions
        self._action_nodes = action_nodes
        # the captured graph is kept (not only its executable) so that the
        # action-reading nodes can be found and retargeted
        self._graph = torch.cuda.CUDAGraph(keep_graph=True)
        stream = torch.cuda.Stream(device=device)  # default priority
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.device(device), torch.cuda.graph(self._graph, stream=stream):
            body()
        torch.cuda.current_stream(device).wait_stream(stream)
        with torch.cuda.device(device):
            self._graph.instantiate()
        self._lib = load_library()
        self._bound = actions  # the tensor the executable reads now

    def _point_at(self, actions: torch.Tensor | None) -> None:
        target = self.actions if actions is None else actions
        if target is self._bound:
            return
        if actions is not None:
            ref = self.actions
            if not actions.is_cuda or actions.device != ref.device:
                raise ValueError("actions must be on the graph's CUDA device")
            if actions.dtype != torch.uint8:
                raise ValueError("actions must use uint8 dtype")
            if actions.shape != ref.shape:
                raise ValueError(f"actions shape must be {list(ref.shape)}")
            if not actions.is_contiguous():
                raise ValueError("actions must be contiguous")
        if target.data_ptr() == self._bound.data_ptr():
            # the same memory (a caching allocator hands a freed block back):
            # the nodes already read it
            self._bound = target
            return
        n = ctypes.c_int32(0)
        check(
            self._lib.jl_graph_retarget_actions(
                int(self._graph.raw_cuda_graph()), int(self._graph.raw_cuda_graph_exec()),
                self.actions.data_ptr(), target.data_ptr(), ctypes.byref(n),
            ),
            "graph action retarget",
        )
        if n.value != self._action_nodes:
            raise RuntimeError(f"graph action retarget changed {n.value} nodes, expected {self._action_nodes}")
        self._bound = target

    def _replay(self, actions: torch.Tensor | None) -> None:
        self._point_at(actions)
        with torch.cuda.device(self._device):
            self._graph.replay()


class MapfGPTResidentGraph(_CapturedStep):
    """One step of the resident MAPF-GPT loop (minimal_p0...:256-281):
    build_tokens_from_state -> append_actions(actions) -> update_actions(actions)
    -> step_sim_only.  Capture after the first (eager) build, so that the
    captured build is the steady-state one; a build that finds changed goals
    still refreshes their fields on replay (the refresh is decided on the
    device)."""

    def __init__(self, sim, builder) -> None:
        self.sim = sim
        self.builder = builder
        actions = torch.zeros_like(sim.actions)

        def body():
            builder.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
            builder.append_actions(actions)
            sim.update_actions(actions)
            sim.step_sim_only()

        steps_before = sim.current_step
        super().__init__(sim.cur_x.device, body, actions, action_nodes=2)
        sim.current_step = steps_before  # capture runs nothing

    def replay(self, actions: torch.Tensor | None = None) -> None:
        """One step with `actions` (uint8 [E, A] on the device), or with the
        graph's own ``actions`` buffer when None."""
        self._replay(actions)
        self.sim.current_step += 1


class MagatStatefulGraph(_CapturedStep):
    """One MAGAT stateful step (grid_world_simulator.cpp:694-785):
    update_actions(actions) -> step_sim_only -> update_derived_state ->
    build_magat_plus_nodes -> finalize_magat_plus_graph.  Capture after the
    first step (whose derived-state pass rebuilds every energy field); later
    steps refresh the fields of changed goals, decided on the device."""

    def __init__(self, sim) -> None:
        if sim.current_step < 1:
            raise RuntimeError("run one eager step before capturing the MAGAT step")
        self.sim = sim
        actions = torch.zeros_like(sim.actions)

        def body():
            sim.update_actions(actions)
            sim.step_sim_only()
            sim.update_derived_state()
            sim.build_magat_plus_nodes()
            sim.finalize_magat_plus_graph()

        steps_before = sim.current_step
        super().__init__(sim.cur_x.device, body, actions, action_nodes=1)
        sim.current_step = steps_before  # capture runs nothing

    def replay(self, actions: torch.Tensor | None = None) -> None:
        """One step with `actions` (uint8 [E, A] on the device), or with the
        graph's own ``actions`` buffer when None."""
        self._replay(actions)
        self.sim.current_step += 1
