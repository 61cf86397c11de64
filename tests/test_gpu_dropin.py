"""The drop-in module ``grid_world_cpp`` as the reference's callers import and
drive it, under MAPF_CUDA_MAP_PROFILE, against the C oracle.

Each test sets MAPF_CUDA_MAP_PROFILE, imports ``grid_world_cpp as ext`` afresh
(the module reads the variable when it is imported, as the reference's build
reads it when it compiles: setup.py:9-40, bind.cpp:95-96), pads smaller maps
into the profile with the one-cell obstacle fence of
``embed_obstacles_in_compiled_profile`` (profiled_topology_loader.py:235-301,
used by grids.py:18-34), and replays one caller's own sequence of calls and
attribute reads:

* the p0 resident loop (minimal_p0_mapf_gpt_resident_runner.py:63-90 and
  256-281): ``build_tokens_from_state`` on the simulator's tensors,
  ``active_mask`` and the done flags masking the actions with
  ``masked_fill_``, ``append_actions``, ``update_actions``, ``step_sim_only``;
* ``PyGBatchBuilder.build`` (fixed_magat_plus_runtime.py:45-115) after
  ``GPUComputeHandler.process_batch`` (expert_running.py:537-548):
  ``update_derived_state`` of the reset rows, the raw batch refresh,
  ``materialize_pyg_inputs``, ``pyg_x[:n].view(n, 4, 13, 13)``, the
  ``arange < num_edges`` mask over the edge storage, ``pyg_batch``/``pyg_ptr``;
* ``view_stateful_outputs`` after the stateful step (a4_runtime.py:285-300,
  fixed_magat_plus_runtime.py:188-227);
* ``MapfGPTRuntimeAdapter.train_step``'s builder reads
  (mapf_gpt_runtime.py:511-541): ``build_tokens``, ``diagnostics``, the
  ``active_mask`` sum and the masked labels.

The 96x96 profile is the smallest that holds the reference's 65x65 mazes with
their fence; its rows (96 columns, three bitmap words) end in half a 64-bit
word, and its 9,216 cells take the two-launch build.
"""
import importlib
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture
def dropin(monkeypatch):
    """Imports grid_world_cpp under a given MAPF_CUDA_MAP_PROFILE; the module
    that was imported before (if any) is restored afterwards."""

    def load(profile_text):
        monkeypatch.setenv("MAPF_CUDA_MAP_PROFILE", profile_text)
        monkeypatch.delitem(sys.modules, "grid_world_cpp", raising=False)
        return importlib.import_module("grid_world_cpp")

    return load


def embed(obstacles, W, H):
    """A real map padded into a WxH profile: obstacles where the map has them,
    a fence of obstacles on the row and column just past the real extent
    (and their corner), free cells beyond (profiled_topology_loader.py:235-261)."""
    rw, rh = obstacles.shape
    out = np.zeros((W, H), np.int32)
    out[:rw, :rh] = obstacles
    if rw < W:
        out[rw, :rh] = 1
    if rh < H:
        out[:rw, rh] = 1
    if rw < W and rh < H:
        out[rw, rh] = 1
    return out, (rw, rh)


def real_maps(kind, E, rw, rh, A, seed):
    from iclr_2027_jointoom_amd.synthetic import iid_grid, maze_grid, place_agents

    rng = np.random.default_rng(seed)
    maps, starts, goals = [], [], []
    for _ in range(E):
        g = maze_grid(rng, rw, rh) if kind == "maze" else iid_grid(rng, rw, rh, 0.2)
        s, t = place_agents(rng, g, A)
        maps.append(g)
        starts.append(s)
        goals.append(t)
    return maps, np.stack(starts), np.stack(goals)


def stack_for_profile(ext, maps):
    """stack_grids_for_compiled_simulator (grids.py:18-34): every map embedded
    in the profile, int32 [E, W, H] on the device, extents int32 [E, 2]."""
    embedded, extents = zip(*(embed(m, ext.COMPILED_MAP_W, ext.COMPILED_MAP_H) for m in maps))
    grids = np.stack(embedded)
    return grids, torch.from_numpy(grids).to(DEV).contiguous(), torch.tensor(extents, dtype=torch.int32, device=DEV)


CASES = [("64x64", "iid", 50, 60), ("96x96", "maze", 65, 65)]


@pytest.mark.parametrize("profile_text,kind,rw,rh", CASES)
def test_p0_resident_loop(dropin, oracle, profile_text, kind, rw, rh):
    """C1-sized rollout (64 agents, 128 steps of a seeded random policy) on
    maps embedded in the profile, horizon 100 so the done mask takes over;
    tokens, the active mask, the masked actions, positions and done flags
    equal the oracle's at every step, and the diagnostics stay zero."""
    ext = dropin(profile_text)
    W, H = (int(v) for v in profile_text.split("x"))
    assert (ext.COMPILED_MAP_W, ext.COMPILED_MAP_H) == (W, H)
    E, A, steps, horizon = 3, 64, 128, 100
    maps, starts, goals = real_maps(kind, E, rw, rh, A, seed=W + rw)
    grids, grids_dev, extents = stack_for_profile(ext, maps)

    # _build_resident_components (minimal_p0...py:63-90)
    sim = ext.GridWorldSimulator(grids_dev, A, 0, int(grids_dev.shape[0] * grids_dev.shape[1] * grids_dev.shape[2]),
                                 20260728, "standard_mapf", horizon)
    sim.set_real_map_extents(extents)
    sim.load_state(torch.as_tensor(starts, device=DEV).contiguous(), torch.as_tensor(goals, device=DEV).contiguous(),
                   torch.zeros((E, A), dtype=torch.uint8, device=DEV), torch.zeros(E, dtype=torch.int32, device=DEV))
    builder = ext.MapfGPTObservationBuilder(grids_dev, A)
    builder.reset_histories()

    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=horizon)
    osim.load_state(starts, goals)
    ob = oracle.OracleMapfGPT(grids, A)
    rng = np.random.default_rng(11)
    actions_flat = torch.empty(E * A, dtype=torch.uint8, device=DEV)
    actions = actions_flat.view(E, A)
    trajectory = torch.empty((steps, E, A), dtype=torch.uint8, device=DEV)
    for step in range(steps):
        builder.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        ob.build_state(osim.cur_x.view(np.int16), osim.cur_y.view(np.int16),
                       osim.goal_x.view(np.int16), osim.goal_y.view(np.int16))
        policy = rng.integers(0, 5, (E, A), dtype=np.uint8)
        actions_flat.copy_(torch.from_numpy(policy.reshape(-1)))  # the policy writes actions_flat
        active_envs = ~(sim.terminated.to(torch.bool) | sim.truncated.to(torch.bool))
        active_agents = builder.active_mask.view(E, A) & active_envs[:, None]
        actions.masked_fill_(~active_agents, 0)
        trajectory[step].copy_(actions)
        builder.append_actions(actions)
        sim.update_actions(actions)
        sim.step_sim_only()

        o_active = (ob.active_mask.reshape(E, A) != 0) & ~((osim.terminated != 0) | (osim.truncated != 0))[:, None]
        o_actions = np.where(o_active, policy, 0).astype(np.uint8)
        ob.append(o_actions)
        osim.step(o_actions)
        torch.cuda.synchronize()
        tag = f"{profile_text} step {step}"
        assert np.array_equal(builder.tokens.cpu().numpy(), ob.tokens), tag
        assert np.array_equal(builder.active_mask.cpu().numpy(), ob.active_mask.astype(bool)), tag
        assert np.array_equal(trajectory[step].cpu().numpy(), o_actions), tag
        assert np.array_equal(torch.stack((sim.cur_x, sim.cur_y), -1).cpu().numpy(), osim.positions()), tag
        assert np.array_equal(sim.terminated.cpu().numpy(), osim.terminated), tag
        assert np.array_equal(sim.truncated.cpu().numpy(), osim.truncated), tag
    assert builder.diagnostics.cpu().tolist() == [0, 0, 0, 0]
    assert int(sim.truncated.sum().item()) + int(sim.terminated.sum().item()) == E  # every env ended
    # no agent ever entered the fence or the free region beyond it
    pos = osim.positions()
    assert (pos[..., 0] < rw).all() and (pos[..., 1] < rh).all()


def _rollout_rows(oracle, grids, extent, starts, goals, A, stages, seed):
    """Raw 8-column rows (env, agent, x, y, gx, gy, action, reset) of a
    standard-MAPF rollout: stage 0 starts the episode (every reset flag 1),
    then one step per stage; at stage 3 the first four agents of every env get
    new goals on free cells inside the real extent (the map's one component),
    with reset flag 1."""
    from iclr_2027_jointoom_amd.synthetic import random_actions

    E = grids.shape[0]
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=64)
    osim.load_state(starts, goals)
    acts = random_actions(np.random.default_rng(seed), stages, E, A)
    rng = np.random.default_rng(seed + 1)
    out = []
    gl = goals.astype(np.int16).copy()
    for s in range(stages):
        rows = osim.state_packed.view(np.int16).reshape(E, A, 8).copy()
        rows[:, :, 4:6] = gl
        rows[:, :, 6] = acts[s]
        rows[:, :, 7] = 1 if s == 0 else 0
        if s == 3:
            for e in range(E):
                free = np.argwhere(grids[e][: extent[0], : extent[1]] == 0)
                gl[e, :4] = free[rng.choice(len(free), 4, replace=False)]
            rows[:, :4, 4:6] = gl[:, :4]
            rows[:, :4, 7] = 1
        out.append(rows.reshape(E * A, 8))
        osim.step(acts[s])
    return out


@pytest.mark.parametrize("profile_text,kind,rw,rh", CASES)
def test_pyg_batch_builder_build_after_process_batch(dropin, oracle, profile_text, kind, rw, rh):
    """Six stages through GPUComputeHandler.process_batch and
    PyGBatchBuilder.build(materialize_edges=True); node features, labels,
    arrival, the masked edge list and the batch vectors equal the oracle's."""
    ext = dropin(profile_text)
    E, A = 3, 48
    maps, starts, goals = real_maps(kind, E, rw, rh, A, seed=7 + rw)
    grids, grids_dev, _ = stack_for_profile(ext, maps)
    sim = ext.StatelessGridWorldSimulator(grids_dev, A, 3)
    m = oracle.OracleMagat(grids, A)
    for s, rows in enumerate(_rollout_rows(oracle, grids, (rw, rh), starts, goals, A, 6, seed=rw)):
        full_batch = torch.from_numpy(rows).to(DEV)
        # GPUComputeHandler.filter_reset_agents + process_batch
        agents_to_update = full_batch[full_batch[:, 7] != 0]
        if agents_to_update.shape[0] > 0:
            sim.update_derived_state(agents_to_update, agents_to_update.shape[0])
        sim.refresh_compact_state_from_raw_batch(full_batch)
        # PyGBatchBuilder.build
        sim.materialize_pyg_inputs()
        num_nodes = full_batch.shape[0]
        x = sim.pyg_x[:num_nodes].view(num_nodes, 4, 13, 13)
        y = full_batch[:, 6].to(dtype=torch.long)
        arrived = (full_batch[:, 2] == full_batch[:, 4]) & (full_batch[:, 3] == full_batch[:, 5])
        edge_index_storage = sim.pyg_edge_index_storage
        edge_attr_storage = sim.pyg_edge_attr_storage
        num_edges = sim.pyg_num_edges
        total_capacity = edge_attr_storage.shape[0]
        valid_mask = torch.arange(total_capacity, device=edge_attr_storage.device,
                                  dtype=num_edges.dtype) < num_edges.reshape(())
        edge_index, edge_attr = edge_index_storage[:, valid_mask], edge_attr_storage[valid_mask]

        reset_rows = rows[rows[:, 7] != 0]
        if len(reset_rows):
            m.update_energy(reset_rows.view(np.uint16), len(reset_rows))
        m.refresh(rows.view(np.uint16))
        m.nodes()
        m.edges()
        tag = f"{profile_text} stage {s}"
        assert np.array_equal(x.cpu().numpy(), m.pyg_x.reshape(num_nodes, 4, 13, 13)), tag
        ei, ea = m.valid_edges()
        assert ei.shape[1] > 0, tag
        assert np.array_equal(edge_index.cpu().numpy(), ei), tag
        assert np.array_equal(edge_attr.cpu().numpy(), ea), tag
        assert np.array_equal(y.cpu().numpy(), rows[:, 6].astype(np.int64)), tag
        assert np.array_equal(arrived.cpu().numpy(), (rows[:, 2:4] == rows[:, 4:6]).all(1)), tag
        assert torch.equal(sim.pyg_batch.cpu(), torch.arange(E).repeat_interleave(A)), tag
        assert torch.equal(sim.pyg_ptr.cpu(), torch.arange(E + 1) * A), tag
        assert np.array_equal(sim.energy_maps.cpu().numpy(), m.energy), tag


@pytest.mark.parametrize("profile_text,kind,rw,rh", CASES)
def test_view_stateful_outputs_after_the_stateful_step(dropin, oracle, profile_text, kind, rw, rh):
    """a4_runtime.py:285-300: update_actions, step_sim_only,
    update_derived_state, build_magat_plus_inputs, then
    view_stateful_outputs' reads (pyg_x.view, actions as labels, arrival from
    the simulator's positions and goals, the masked edges)."""
    from iclr_2027_jointoom_amd.synthetic import random_actions

    ext = dropin(profile_text)
    E, A, steps = 2, 48, 4
    maps, starts, goals = real_maps(kind, E, rw, rh, A, seed=3 + rw)
    grids, grids_dev, extents = stack_for_profile(ext, maps)
    sim = ext.GridWorldSimulator(grids_dev, A, 0, E * grids.shape[1] * grids.shape[2], 5, "standard_mapf", 64)
    sim.set_real_map_extents(extents)
    sim.load_state(torch.from_numpy(starts).to(DEV), torch.from_numpy(goals).to(DEV),
                   torch.zeros((E, A), dtype=torch.uint8, device=DEV), torch.zeros(E, dtype=torch.int32, device=DEV))
    osim = oracle.OracleSim(grids, A, task_mode=1, max_episode_steps=64)
    osim.load_state(starts, goals)
    acts = random_actions(np.random.default_rng(2), steps, E, A)
    for s in range(steps):
        sim.update_actions(torch.from_numpy(acts[s]).to(DEV))
        sim.step_sim_only()
        sim.update_derived_state()
        sim.build_magat_plus_inputs()
        osim.step(acts[s])
        num_nodes = sim.pyg_x.shape[0]
        x = sim.pyg_x.view(num_nodes, 4, 13, 13)
        y = sim.actions.reshape(-1).to(dtype=torch.long)
        arrived = (sim.cur_x.reshape(-1)[:num_nodes] == sim.goal_x.reshape(-1)[:num_nodes]) & (
            sim.cur_y.reshape(-1)[:num_nodes] == sim.goal_y.reshape(-1)[:num_nodes])
        num_edges = sim.pyg_num_edges
        valid = torch.arange(sim.pyg_edge_attr_storage.shape[0], device=DEV, dtype=num_edges.dtype) < num_edges.reshape(())
        edge_index = sim.pyg_edge_index_storage[:, valid]

        rows = osim.state_packed.copy()
        rows_reset = rows.copy()
        rows_reset[:, 7] = 1
        m = oracle.OracleMagat(grids, A)
        m.update_energy(rows_reset, len(rows_reset))
        m.refresh(rows)
        m.nodes()
        m.edges()
        tag = f"{profile_text} step {s}"
        assert np.array_equal(x.cpu().numpy(), m.pyg_x.reshape(num_nodes, 4, 13, 13)), tag
        assert np.array_equal(edge_index.cpu().numpy(), m.valid_edges()[0]), tag
        assert np.array_equal(y.cpu().numpy(), acts[s].reshape(-1).astype(np.int64)), tag
        pos, gol = osim.positions().reshape(-1, 2), np.stack([osim.goal_x, osim.goal_y], -1).reshape(-1, 2)
        assert np.array_equal(arrived.cpu().numpy(), (pos == gol.astype(np.int16)).all(1)), tag


@pytest.mark.parametrize("profile_text,kind,rw,rh", CASES)
def test_mapf_gpt_runtime_train_step_reads(dropin, oracle, profile_text, kind, rw, rh):
    """MapfGPTRuntimeAdapter.train_step (mapf_gpt_runtime.py:511-541) over
    four 13-column stages of a rollout: build_tokens, the diagnostics copied
    into the stage statistics with the active count, tokens, and the labels
    of inactive agents masked to -1 in a reused workspace."""
    ext = dropin(profile_text)
    E, A = 3, 64
    maps, starts, goals = real_maps(kind, E, rw, rh, A, seed=5 + rw)
    grids, grids_dev, _ = stack_for_profile(ext, maps)
    builder = ext.MapfGPTObservationBuilder(grids_dev, A)
    ob = oracle.OracleMapfGPT(grids, A)
    stage_stats = torch.empty(5, dtype=torch.int64, device=DEV)
    workspace = None
    history = np.full((E * A, 5), 5, np.uint16)
    for s, rows8 in enumerate(_rollout_rows(oracle, grids, (rw, rh), starts, goals, A, 4, seed=rw + 1)):
        rows = np.zeros((E * A, 13), np.uint16)
        rows[:, :8] = rows8.view(np.uint16)
        rows[:, 8:13] = history
        raw_stage = torch.from_numpy(rows.view(np.int16)).to(DEV)

        builder.build_tokens(raw_stage)
        stage_stats[:4].copy_(builder.diagnostics)
        stage_stats[4] = builder.active_mask.sum(dtype=torch.int64)
        stats = stage_stats.detach().cpu().tolist()
        assert not any(stats[:4]), stats
        assert int(builder.tokens.shape[0]) == E * A
        if workspace is None or workspace.shape != builder.labels.shape or workspace.device != builder.labels.device:
            workspace = torch.empty_like(builder.labels)
        labels = workspace
        labels.copy_(builder.labels)
        labels.masked_fill_(~builder.active_mask, -1)

        ob.build_rows(rows)
        tag = f"{profile_text} stage {s}"
        active = ob.active_mask.astype(bool)
        assert stats[4] == int(active.sum()), tag
        assert np.array_equal(builder.tokens.cpu().numpy(), ob.tokens), tag
        assert np.array_equal(labels.cpu().numpy(), np.where(active, ob.labels, -1)), tag
        history[:, :-1] = history[:, 1:]
        history[:, -1] = rows[:, 6]
