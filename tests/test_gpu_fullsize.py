"""Full BASELINE sizes that the other GPU tests reach only at smaller shapes.

* C3 (1024 envs x 128 agents, 64x64 recursive-backtracker mazes) with every
  goal fresh: 131,072 BFS fields in one build (mapf_gpt_cuda.cu:181-325),
  single-launch and two-launch builds equal bit for bit, three sampled envs
  equal to the oracle, and properties over every agent (distance 0 at the
  goal, the ego's own slot and window centre).
* C5 (256 envs x 1024 agents, 256x256 warehouses) compact records through the
  ring: CompactRingBuffer -> CompactDMAWorker (the native per-stage upload and
  expansion) -> MapfGPTOnlinePipeline -> build_tokens
  (frozen_stage_source.py:105-156, expert_running.py:463-531,
  mapf_gpt_online.py:97-184); the expanded 13-column rows and the tokens of
  three sampled envs equal the oracle's, over a first stage that starts every
  episode and a second that starts new episodes in every seventh env.
"""
import time

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def test_c3_full_size_fresh_maze_build(oracle):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = 1024, 64, 128
    print("[c3 fresh] generating 1024 mazes", flush=True)
    grids, starts, goals = make_batch(2030, E, W, W, A, kind="maze")
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).cuda()
    one = ext.MapfGPTObservationBuilder(g, A)
    two = ext.MapfGPTObservationBuilder(g, A)
    two._desc.build_scratch = None  # the two-launch build
    assert one.single_launch and not two.single_launch
    state = [torch.from_numpy(np.ascontiguousarray(v)).cuda()
             for v in (starts[..., 0], starts[..., 1], goals[..., 0], goals[..., 1])]
    one.build_tokens_from_state(*state)
    two.build_tokens_from_state(*state)
    torch.cuda.synchronize()
    for name in ("tokens", "active_mask", "cost_to_go", "state_packed", "diagnostics"):
        assert torch.equal(getattr(one, name), getattr(two, name)), name
    assert one.diagnostics.cpu().tolist() == [0, 0, 0, 0]
    sample = [0, 333, 1023]
    ob = oracle.OracleMapfGPT(grids[sample], A)
    ob.build_state(*(v.cpu().numpy()[sample] for v in state))
    tok = one.tokens.view(E, A, 256)
    assert np.array_equal(tok[sample].cpu().numpy().reshape(-1, 256), ob.tokens)
    assert np.array_equal(one.cost_to_go[sample].cpu().numpy().view(np.uint16), ob.cost_to_go)
    # every agent: its field is 0 at its goal; its own slot (relative position
    # 0 -> token 20) and its window centre (d - d = 0 -> 20); the starts lie on
    # the goals' component, so every ego is reachable
    ctg = one.cost_to_go
    e_idx = torch.arange(E, device="cuda")[:, None].expand(E, A)
    a_idx = torch.arange(A, device="cuda")[None, :].expand(E, A)
    at_goal = ctg[e_idx, a_idx, state[2].long(), state[3].long()]
    assert bool((at_goal == 0).all())
    assert bool((tok[:, :, 121] == 20).all() and (tok[:, :, 122] == 20).all() and (tok[:, :, 60] == 20).all())


def _c5_compact_records(E, W, A, seed):
    """Two stages of compact records on warehouse maps: every episode starts
    at stage 0; at stage 1 every seventh env starts a new episode with its
    goal set rolled by five agents."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals0 = make_batch(seed, E, W, W, A, kind="warehouse")
    rng = np.random.default_rng(seed)
    N = E * A
    positions = np.stack([starts.reshape(N, 2), np.roll(starts, 1, axis=1).reshape(N, 2)]).astype(np.uint16)
    actions = rng.integers(0, 5, size=(2, N)).astype(np.uint8)
    episode_starts = np.zeros((2, E), np.uint8)
    episode_starts[0] = 1
    episode_starts[1, ::7] = 1
    stage_goals = np.stack([goals0, np.roll(goals0, 5, axis=1)]).astype(np.uint16)  # [2, E, A, 2]
    return grids, positions, actions, episode_starts, stage_goals


def test_c5_compact_stages_through_the_ring(oracle):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.ring import MapfGPTOnlinePipeline
    from oracle.records import expand_records

    E, W, A = 256, 256, 1024
    N = E * A
    print("[c5 ring] generating 256 warehouse maps and two compact stages", flush=True)
    grids, positions, actions, episode_starts, stage_goals = _c5_compact_records(E, W, A, 2031)
    sample = [5, 128, 255]
    builder = profile(W, W).MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)

    class Keep:
        """MapfGPTRuntimeAdapter.train_step's reads, keeping the sampled envs."""

        def __init__(self):
            self.stages, self.tokens, self.diag = [], [], []

        def train_step(self, b, raw_stage):
            b.build_tokens(raw_stage)
            rows = raw_stage.view(E, A, 13)
            self.stages.append(rows[sample].cpu().numpy())
            self.tokens.append(b.tokens.view(E, A, 256)[sample].cpu().numpy())
            self.diag.append(b.diagnostics.cpu().tolist())
            tok = b.tokens.view(E, A, 256)
            assert bool((tok[:, :, 121] == 20).all() and (tok[:, :, 60] == 20).all())
            return {"rows": int(raw_stage.shape[0])}

    runtime = Keep()
    pipe = MapfGPTOnlinePipeline(builder, runtime, capacity=2 * N, batch_threshold=N,
                                 record_format="compact").initialize()
    for s in range(2):
        pipe.ring_buffer.write_compact(0, positions[s], actions[s], episode_starts[s],
                                       goals=stage_goals[s].reshape(N, 2))
    pipe.dma_worker_loop()
    deadline = time.monotonic() + 120
    try:
        while len(runtime.tokens) < 2:
            if pipe.consume_once() is None:
                assert time.monotonic() < deadline, pipe.get_stats()
                time.sleep(0.001)
    finally:
        pipe.shutdown()
    assert runtime.diag == [[0, 0, 0, 0]] * 2
    stats = pipe.get_stats()
    assert stats["compute_ptr"] == 2 * N and stats["env_write_stage"] == [2] * E
    for k, e in enumerate(sample):
        lo, hi = e * A, (e + 1) * A
        starts_e = episode_starts[:, [e]]
        goals_e = np.stack([stage_goals[s, e] for s in range(2) if starts_e[s, 0]])
        rows = expand_records(positions[:, lo:hi], actions[:, lo:hi], starts_e, goals_e, 1, 13)
        ob = oracle.OracleMapfGPT(grids[e:e + 1], A)
        for s in range(2):
            got = runtime.stages[s][k].view(np.uint16).copy()
            assert np.all(got[:, 0] == e)
            got[:, 0] = 0  # the single-env oracle's env id
            assert np.array_equal(got, rows[s]), (e, s)
            ob.build_rows(rows[s])
            assert np.array_equal(runtime.tokens[s][k], ob.tokens), (e, s)
