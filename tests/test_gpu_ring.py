"""GPU tests of the expert-record ring: producers -> shared ring -> pinned
staging -> HBM ring -> MapfGPTObservationBuilder / MAGAT simulator, every
consumed stage checked against the C oracle fed the same rows
(mapf_gpt_online.py:97-184, expert_running.py:602-779)."""
import threading
import time

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _stages(E, A, S, W, features, seed):
    """S stages of env-major rows on one seeded map per env, agents moving randomly."""
    from iclr_2027_jointoom_amd.synthetic import make_batch

    grids, starts, goals = make_batch(seed, E, W, W, A)
    rng = np.random.default_rng(seed)
    stages = np.zeros((S, E * A, features), np.uint16)
    pos = starts.astype(np.int64)
    for s in range(S):
        blk = stages[s].reshape(E, A, features)
        blk[:, :, 0] = np.arange(E)[:, None]
        blk[:, :, 1] = np.arange(A)[None]
        blk[:, :, 2:4] = pos
        blk[:, :, 4:6] = goals
        blk[:, :, 6] = rng.integers(0, 5, size=(E, A))
        blk[:, :, 7] = 1 if s == 0 else (rng.random((E, A)) < 0.05)
        if features == 13:
            blk[:, :, 8:13] = rng.integers(0, 6, size=(E, A, 5))
        pos = np.roll(pos, 1, axis=1)  # distinct cells, still on the free component
    return grids, stages


def _produce(ring, stages, E, A):
    def worker(e):
        for st in stages:
            ring.reserve_and_write(np.array(st[e * A:(e + 1) * A], copy=True))

    threads = [threading.Thread(target=worker, args=(e,), daemon=True) for e in range(E)]
    for t in threads:
        t.start()
    return threads


class _TokenRuntime:
    """Stand-in for MapfGPTRuntimeAdapter.train_step: build tokens, keep a copy."""

    def __init__(self):
        self.tokens = []

    def train_step(self, builder, raw_stage):
        builder.build_tokens(raw_stage)
        self.tokens.append(builder.tokens.clone())
        return {"rows": int(raw_stage.shape[0])}


def test_mapf_gpt_online_pipeline_streams_stages_into_tokens(oracle):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.ring import MapfGPTOnlinePipeline

    E, A, S, W = 4, 32, 6, 32
    grids, stages = _stages(E, A, S, W, 13, seed=21)
    builder = profile(W, W).MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)
    runtime = _TokenRuntime()
    pipe = MapfGPTOnlinePipeline(builder, runtime, capacity=3 * E * A, batch_threshold=E * A).initialize()
    pipe.dma_worker_loop()
    threads = _produce(pipe.ring_buffer, stages, E, A)
    deadline = time.monotonic() + 60
    try:
        while len(runtime.tokens) < S:
            if pipe.consume_once(capture_stage_hash=len(runtime.tokens) == 0) is None:
                assert time.monotonic() < deadline, pipe.get_stats()
                time.sleep(0.001)
    finally:
        pipe.shutdown()
    for t in threads:
        t.join(timeout=5)
    ob = oracle.OracleMapfGPT(grids, A)
    for s in range(S):
        ob.build_rows(stages[s])
        assert np.array_equal(runtime.tokens[s].cpu().numpy(), ob.tokens), s
    stats = pipe.get_stats()
    assert stats["compute_ptr"] == S * E * A and stats["env_write_stage"] == [S] * E


def test_extreme_pipeline_magat_stages_match_oracle(oracle):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.ring import ExtremeMAPFPipeline

    E, A, S, W = 3, 48, 4, 64
    grids, stages = _stages(E, A, S, W, 8, seed=5)
    sim = profile(W, W).StatelessGridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 3)
    pipe = ExtremeMAPFPipeline(sim, capacity=2 * E * A, batch_threshold=E * A).initialize()
    assert pipe.stage_mode and pipe.graph_rows == E * A
    pipe.dma_worker_loop()
    threads = _produce(pipe.ring_buffer, stages, E, A)
    m = oracle.OracleMagat(grids, A)
    deadline = time.monotonic() + 60
    try:
        for s in range(S):
            x = None
            while x is None:
                x = pipe.train_step()
                if x is None:
                    assert time.monotonic() < deadline, pipe.get_stats()
                    time.sleep(0.001)
            # train_step refreshes energy + occupancy; the nodes and the graph are
            # built by the MAGAT runtime's PyGBatchBuilder (fixed_magat_plus_runtime.py:83-115)
            sim.materialize_pyg_inputs()
            x = sim.pyg_x
            rows = stages[s]
            reset = rows[rows[:, 7] != 0]
            m.update_energy(reset, len(reset))
            m.refresh(rows)
            m.nodes()
            m.edges()
            torch.cuda.synchronize()
            assert np.array_equal(x.cpu().numpy(), m.pyg_x), s
            assert np.array_equal(sim.pyg_edge_index.cpu().numpy(), m.valid_edges()[0]), s
    finally:
        pipe.shutdown()
    for t in threads:
        t.join(timeout=5)


def test_pipeline_rejects_mismatched_threshold():
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.ring import MapfGPTOnlinePipeline

    builder = profile(32, 32).MapfGPTObservationBuilder(torch.zeros((2, 32, 32), dtype=torch.int32).cuda(), 4)
    with pytest.raises(ValueError, match="one complete frontier"):
        MapfGPTOnlinePipeline(builder, _TokenRuntime(), capacity=16, batch_threshold=4).initialize()
