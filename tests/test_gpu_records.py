"""GPU tests of compact expert records: jl_expand_records against the CPU
restatement of the producers' rows (oracle/records.py), and the compact ring
(producer processes -> CompactRingBuffer -> CompactDMAWorker -> device
expansion -> the builders) against the row ring on the same archive."""
import time

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from oracle.records import expand_records  # noqa: E402
from records_data import make_compact  # noqa: E402


@pytest.mark.parametrize("features", [13, 8])
@pytest.mark.parametrize("E,A,S,offset", [(3, 100, 9, 0), (2, 1024, 4, 0), (5, 7, 6, 1), (1, 300, 3, 3)])
def test_expand_records_matches_oracle(features, E, A, S, offset):
    from iclr_2027_jointoom_amd.records import RecordExpander

    print(f"[records] E={E} A={A} S={S} F={features} row offset={offset}", flush=True)
    _, (pos, act, st, goals) = make_compact(40 + E, E, 64 if A < 1024 else 128, A, S)
    want = expand_records(pos, act, st, goals, E, features)
    N = E * A
    exp = RecordExpander(E, A, features, "cuda:0")
    # rows at an offset of `offset` rows: 16-byte aligned only for offset 0
    out = torch.full((N + offset, features), -1, dtype=torch.int16, device="cuda")
    rows = out[offset:]
    gidx = np.cumsum(st.reshape(-1)).reshape(st.shape) - 1
    for s in range(S):
        new_goals = np.zeros((E, A, 2), np.uint16)
        for e in np.flatnonzero(st[s]):
            new_goals[e] = goals[gidx[s, e]]
        dev = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.int16) if x.dtype == np.uint16 else
                                         np.ascontiguousarray(x)).cuda()
        exp.expand(dev(pos[s]), dev(act[s]), dev(st[s]), dev(new_goals.reshape(N, 2)), rows)
        torch.cuda.synchronize()
        got = rows.cpu().numpy().view(np.uint16)
        assert np.array_equal(got, want[s]), s
    if offset:
        assert torch.all(out[:offset] == -1)


def test_expand_records_rejects_bad_tensors():
    from iclr_2027_jointoom_amd.records import RecordExpander

    exp = RecordExpander(2, 4, 13, "cuda:0")
    ok = dict(positions=torch.zeros((8, 2), dtype=torch.int16, device="cuda"),
              actions=torch.zeros(8, dtype=torch.uint8, device="cuda"),
              episode_start=torch.ones(2, dtype=torch.uint8, device="cuda"),
              new_goals=torch.zeros((8, 2), dtype=torch.int16, device="cuda"),
              rows=torch.zeros((8, 13), dtype=torch.int16, device="cuda"))
    bad = dict(ok, rows=torch.zeros((8, 8), dtype=torch.int16, device="cuda"))
    with pytest.raises(RuntimeError, match="shape"):
        exp.expand(**bad)
    bad = dict(ok, actions=torch.zeros(8, dtype=torch.uint8))
    with pytest.raises(RuntimeError, match="contiguous tensor on cuda"):
        exp.expand(**bad)
    exp.expand(**ok)
    torch.cuda.synchronize()


class _TokenRuntime:
    def __init__(self):
        self.tokens = []
        self.labels = []

    def train_step(self, builder, raw_stage):
        builder.build_tokens(raw_stage)
        self.tokens.append(builder.tokens.clone())
        self.labels.append(builder.labels.clone())
        return {"rows": int(raw_stage.shape[0])}


def _run_mapf_gpt(grids, records, E, A, S, record_format, workers):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.ring import MapfGPTOnlinePipeline, RingStageSource

    W = grids.shape[1]
    builder = profile(W, W).MapfGPTObservationBuilder(torch.from_numpy(grids.astype(np.int32)).cuda(), A)
    runtime = _TokenRuntime()
    pipe = MapfGPTOnlinePipeline(builder, runtime, capacity=2 * E * A, batch_threshold=E * A,
                                 record_format=record_format).initialize()
    config = {"num_agents": A, "num_steps": S, "map_names": [f"m{e}" for e in range(E)]}
    src = RingStageSource(pipe.ring_buffer, "mapf_gpt", config, records=records, timeout=60, workers=workers)
    deadline = time.monotonic() + 90
    try:
        src.start()
        pipe.dma_worker_loop()
        while len(runtime.tokens) < S:
            src.check()
            if pipe.consume_once() is None:
                assert time.monotonic() < deadline, pipe.get_stats()
                time.sleep(0.001)
    finally:
        pipe.shutdown()
        src.close()
    return pipe, runtime


def test_compact_mapf_gpt_pipeline_equals_row_pipeline(tmp_path, oracle):
    from iclr_2027_jointoom_amd.records import save_compact_records
    from iclr_2027_jointoom_amd.ring import save_records

    E, A, S, W = 4, 40, 10, 32
    print(f"[records] compact MAPF-GPT pipeline E={E} A={A} S={S}", flush=True)
    grids, arrays = make_compact(23, E, W, A, S, mean_episode=4.0)
    stages = expand_records(*arrays, E, 13)
    save_records(tmp_path / "rows", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    save_compact_records(tmp_path / "compact", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    _, rt_rows = _run_mapf_gpt(grids, tmp_path / "rows", E, A, S, "rows", None)
    pipe, rt_c = _run_mapf_gpt(grids, tmp_path / "compact", E, A, S, "compact", 2)
    ob = oracle.OracleMapfGPT(grids, A)
    for s in range(S):
        assert torch.equal(rt_rows.tokens[s], rt_c.tokens[s]), s
        assert torch.equal(rt_rows.labels[s], rt_c.labels[s]), s
        ob.build_rows(stages[s])
        assert np.array_equal(rt_c.tokens[s].cpu().numpy(), ob.tokens), s
    # bytes over the host link: 5 per agent and step, the flags, and the goal
    # range spanning the envs that start an episode
    goal_bytes = 0
    for s in range(S):
        starting = np.flatnonzero(arrays[2][s])
        goal_bytes += (int(starting[-1]) - int(starting[0]) + 1) * A * 4 if starting.size else 0
    assert pipe.dma_worker.bytes_uploaded == S * (5 * E * A + E) + goal_bytes
    assert pipe.get_stats()["compute_ptr"] == S * E * A


def test_compact_magat_pipeline_equals_row_pipeline(tmp_path):
    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.records import save_compact_records
    from iclr_2027_jointoom_amd.ring import ExtremeMAPFPipeline, RingStageSource, save_records

    E, A, S, W = 3, 48, 6, 64
    print(f"[records] compact MAGAT pipeline E={E} A={A} S={S}", flush=True)
    grids, arrays = make_compact(31, E, W, A, S, mean_episode=3.0)
    stages = expand_records(*arrays, E, 8)
    save_records(tmp_path / "rows", backend="magat", grids=grids, stages=stages, metadata={})
    save_compact_records(tmp_path / "compact", backend="magat", grids=grids, stages=stages, metadata={})
    results = {}
    for fmt, rec, workers in (("rows", tmp_path / "rows", None), ("compact", tmp_path / "compact", 3)):
        sim = profile(W, W).StatelessGridWorldSimulator(torch.from_numpy(grids.astype(np.int32)).cuda(), A, 3)
        pipe = ExtremeMAPFPipeline(sim, capacity=2 * E * A, batch_threshold=E * A, record_format=fmt).initialize()
        config = {"num_agents": A, "num_steps": S, "map_names": [f"m{e}" for e in range(E)]}
        src = RingStageSource(pipe.ring_buffer, "magat", config, records=rec, timeout=60, workers=workers)
        xs = []
        deadline = time.monotonic() + 90
        try:
            src.start()
            pipe.dma_worker_loop()
            while len(xs) < S:
                src.check()
                x = pipe.train_step()
                if x is None:
                    assert time.monotonic() < deadline, pipe.get_stats()
                    time.sleep(0.001)
                    continue
                sim.materialize_pyg_inputs()
                xs.append((sim.pyg_x.clone(), sim.energy_maps.clone() if hasattr(sim, "energy_maps") else None))
        finally:
            pipe.shutdown()
            src.close()
        results[fmt] = xs
    for s in range(S):
        assert torch.equal(results["rows"][s][0], results["compact"][s][0]), s
        if results["rows"][s][1] is not None:
            assert torch.equal(results["rows"][s][1], results["compact"][s][1]), s
