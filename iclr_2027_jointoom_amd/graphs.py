"""HIP-graph capture of the resident loops.

The reference launches every kernel of a step from the host each step
(minimal_p0_mapf_gpt_resident_runner.py:256-281 for the MAPF-GPT loop,
fixed_magat_plus_runtime.py:53-115 with GridWorldSimulator::step_and_build_pyg,
grid_world_simulator.cpp:694-785, for the MAGAT loop).  Here one step of
either loop is captured once into a HIP graph (torch.cuda.CUDAGraph on ROCm)
and replayed: every launch of the step goes to the current stream, none
allocates, synchronises with the host or records a memset node (buffers are
cleared by fill kernels), so the captured step equals the eager one.

A graph reads its inputs from fixed device buffers: the caller writes the
next actions into ``actions`` (a tensor owned by the graph object) before
each ``replay``.  Objects captured in a graph must stay alive and must not be
re-created while the graph is in use.  The host-side step counter of the
simulator is advanced by ``replay`` as an eager step would.
"""
from __future__ import annotations

import torch


class _CapturedStep:
    def __init__(self, device: torch.device, body) -> None:
        self._device = device
        self._graph = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream(device=device)  # default priority
        stream.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.device(device), torch.cuda.graph(self._graph, stream=stream):
            body()
        torch.cuda.current_stream(device).wait_stream(stream)

    def _replay(self) -> None:
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
        self.actions = torch.zeros_like(sim.actions)

        def body():
            builder.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
            builder.append_actions(self.actions)
            sim.update_actions(self.actions)
            sim.step_sim_only()

        steps_before = sim.current_step
        super().__init__(sim.cur_x.device, body)
        sim.current_step = steps_before  # capture runs nothing

    def replay(self) -> None:
        self.sim.current_step += 1
        self._replay()


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
        self.actions = torch.zeros_like(sim.actions)

        def body():
            sim.update_actions(self.actions)
            sim.step_sim_only()
            sim.update_derived_state()
            sim.build_magat_plus_nodes()
            sim.finalize_magat_plus_graph()

        steps_before = sim.current_step
        super().__init__(sim.cur_x.device, body)
        sim.current_step = steps_before  # capture runs nothing

    def replay(self) -> None:
        self.sim.current_step += 1
        self._replay()
