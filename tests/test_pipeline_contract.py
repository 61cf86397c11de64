"""The stage consumer's contract with its runtime backends, on the CPU
(ExtremeMAPFPipeline.train_step, iclr_2027_jointoom_amd/ring.py).

Restates the reference's runtime-path cases of tests/expert/test_pipeline.py
(:988-1636 with mocked stage extraction, :1636-2310 through the real ring and
DMA worker): a train step takes the next complete env-aligned stage, filters
its reset rows, hands both to the GPU handler, then calls the runtime backend
(MAGAT or MAPF-GPT, same signature) with the simulator and the exact stage
tensor, and returns what the backend returns; no stage means no backend call;
a backend error propagates after the stage was consumed and released, and the
ring's counters after each frontier are the reference's.

One deliberate difference: the reference blocks the host on the DMA event
before taking a stage (expert_running.py:728); here the consumer's stream
waits on the stage's upload event on the device, so no host synchronisation
is asserted instead.
"""
import contextlib
from unittest.mock import MagicMock, patch

import numpy as np
import pytest
import torch

from iclr_2027_jointoom_amd.ring import FEATURE_DIM, RESET_FLAG_COL, ExtremeMAPFPipeline


@contextlib.contextmanager
def cpu_device():
    """The pipeline's device calls on the CPU (pinning, streams, events)."""
    with patch("torch.Tensor.pin_memory", lambda self: self), \
            patch("torch.cuda.Stream", side_effect=lambda *a, **k: object()), \
            patch("torch.cuda.Event", side_effect=lambda *a, **k: MagicMock()), \
            patch("torch.cuda.stream", lambda s: contextlib.nullcontext()), \
            patch("torch.cuda.current_stream", lambda *a, **k: object()):
        yield


def two_env_sim():
    sim = MagicMock()
    sim.pyg_ptr = torch.tensor([0, 2, 4], dtype=torch.int64)  # 2 envs x 2 agents
    sim.pyg_batch = torch.zeros(4, dtype=torch.int64)
    return sim


def pipeline_for(sim):
    with cpu_device():
        p = ExtremeMAPFPipeline(sim, capacity=8, batch_threshold=4, device="cpu")
        p.initialize()
    return p


def frontier(reset=(0, 0, 0, 0), positions=((10, 10), (10, 11), (20, 20), (20, 21)), actions=(0, 0, 0, 0)):
    """A 2-env x 2-agent stage: env-major ids, goals 20 cells off."""
    f = torch.zeros((4, FEATURE_DIM), dtype=torch.int16)
    f[:, 0] = torch.tensor([0, 0, 1, 1], dtype=torch.int16)
    f[:, 1] = torch.tensor([0, 1, 0, 1], dtype=torch.int16)
    f[:, 2:4] = torch.tensor(positions, dtype=torch.int16)
    f[:, 4:6] = f[:, 2:4] + 20
    f[:, 6] = torch.tensor(actions, dtype=torch.int16)
    f[:, RESET_FLAG_COL] = torch.tensor(reset, dtype=torch.int16)
    return f


def env_blocks(f, agents=2):
    return [f[k:k + agents].numpy().astype(np.uint16) for k in range(0, f.shape[0], agents)]


class Recorder:
    """A backend's train_step(simulator_or_builder, stage) that records its calls."""

    def __init__(self, backend, fail_on=None, extra=None):
        self.backend, self.fail_on, self.extra = backend, fail_on, extra
        self.calls = []

    def train_step(self, target, stage):
        self.calls.append((target, stage.clone()))
        if self.fail_on == len(self.calls):
            raise RuntimeError(f"{self.backend} frontier failure")
        out = {"backend": self.backend, "rows": int(stage.shape[0])}
        if self.extra is not None:
            out.update(self.extra(self, stage))
        return out


def mocked_stage(pipeline, *stages, reset_subsets=None):
    """Stage extraction and the GPU handler replaced by mocks (the reference's
    :1053-1636 setup)."""
    pipeline.dma_worker = MagicMock()
    pipeline.dma_event = MagicMock()
    pipeline.extract_env_aligned_batch = MagicMock(side_effect=list(stages))
    pipeline.gpu_handler = MagicMock()
    if reset_subsets is None:
        reset_subsets = [s[:0] if s is not None else None for s in stages]
    pipeline.gpu_handler.filter_reset_agents.side_effect = list(reset_subsets)


# ---- construction and the empty cases -------------------------------------------------------------
def test_construction_and_initialize():
    sim = MagicMock()
    sim.pyg_ptr = torch.tensor([0], dtype=torch.int64)  # no env layout: a row ring
    sim.pyg_batch = torch.zeros(0, dtype=torch.int64)
    p = ExtremeMAPFPipeline(sim, capacity=1024, batch_threshold=256, feature_dim=FEATURE_DIM, device="cpu")
    assert (p.capacity, p.batch_threshold, p.feature_dim, p.dma_read_ptr, p.compute_ptr) == (
        1024, 256, FEATURE_DIM, 0, 0)
    with cpu_device():
        p.initialize()
    assert p.ring_buffer is not None and p.gpu_buffer is not None
    assert p.gpu_handler is not None and p.dma_worker is not None
    assert p.reserve_and_write(np.zeros((10, FEATURE_DIM), np.uint16)) == (0, 10)
    assert p.train_step() is None  # a row ring has no stage to take


def test_no_stage_means_no_backend_call():
    sim = two_env_sim()
    assert ExtremeMAPFPipeline(sim, capacity=8, batch_threshold=4, device="cpu").train_step(
        runtime=Recorder("magat")) is None  # not initialised
    p = pipeline_for(sim)
    assert p.train_step() is None  # nothing written
    mocked_stage(p, None)
    rt = Recorder("mapf_gpt")
    assert p.train_step(runtime=rt) is None
    assert rt.calls == []
    p.extract_env_aligned_batch.assert_called_once_with(4, agents_per_env=2, num_envs=2)
    p.gpu_handler.process_batch.assert_not_called()
    p.dma_event.synchronize.assert_not_called()  # the stage wait is on the device


def test_get_stats_exposes_the_stage_counters():
    stats = pipeline_for(two_env_sim()).get_stats()
    assert stats["capacity"] == 8 and stats["stage_rows"] == 4 and stats["num_stage_slots"] >= 1
    for key in ("stage_ready_counts", "stage_seq_tags", "env_write_stage"):
        assert key in stats
    assert (stats["reserve_ptr"], stats["dma_read_ptr"], stats["compute_ptr"]) == (0, 0, 0)


# ---- one stage through mocks ------------------------------------------------------------------------
@pytest.mark.parametrize("backend", ["magat", "mapf_gpt"])
def test_backend_gets_the_simulator_and_the_exact_stage(backend):
    sim = two_env_sim()
    p = pipeline_for(sim)
    stage = frontier()
    mocked_stage(p, stage)
    captured = {}
    rt = Recorder(backend, extra=lambda r, s: captured.update(stage=s) or {})
    assert p.train_step(runtime=rt) == {"backend": backend, "rows": 4}
    target, forwarded = rt.calls[0]
    assert target is sim
    assert captured["stage"] is stage  # the tensor itself, no copy
    assert forwarded.dtype == torch.int16 and forwarded.shape == (4, FEATURE_DIM)
    view = forwarded.view(2, 2, FEATURE_DIM)  # env-major blocks, agent ids 0..1
    assert view[:, :, 0].tolist() == [[0, 0], [1, 1]] and view[:, :, 1].tolist() == [[0, 1], [0, 1]]
    p.extract_env_aligned_batch.assert_called_once_with(4, agents_per_env=2, num_envs=2)


def test_reset_rows_are_filtered_then_processed_then_the_backend_runs():
    p = pipeline_for(two_env_sim())
    stage = frontier(reset=(0, 1, 0, 0))
    subset = stage[1:2]
    mocked_stage(p, stage, reset_subsets=[subset])
    order = []
    p.gpu_handler.filter_reset_agents.side_effect = lambda b: (order.append("filter"), subset)[1]
    p.gpu_handler.process_batch.side_effect = lambda b, s: order.append("process")
    rt = Recorder("magat", extra=lambda r, s: order.append("runtime") or {})
    p.train_step(runtime=rt)
    assert order == ["filter", "process", "runtime"]
    p.gpu_handler.filter_reset_agents.assert_called_once_with(stage)
    p.gpu_handler.process_batch.assert_called_once_with(stage, subset)


def test_empty_reset_subset_still_goes_through_the_handler():
    p = pipeline_for(two_env_sim())
    stage = frontier()
    mocked_stage(p, stage)
    p.train_step(runtime=Recorder("magat"))
    processed, subset = p.gpu_handler.process_batch.call_args.args
    assert torch.equal(processed, stage) and subset.shape == (0, FEATURE_DIM)


def test_backend_errors_propagate_after_the_handler_ran():
    p = pipeline_for(two_env_sim())
    mocked_stage(p, frontier())

    class Failing:
        def train_step(self, simulator, batch):
            raise RuntimeError("backend failure")

    with pytest.raises(RuntimeError, match="backend failure"):
        p.train_step(runtime=Failing())
    p.gpu_handler.process_batch.assert_called_once()


def test_any_backend_with_the_signature_and_one_simulator_for_all():
    sim = two_env_sim()
    p = pipeline_for(sim)
    stage = frontier()
    mocked_stage(p, stage, stage, stage, stage)

    class A:
        def train_step(self, simulator, batch):
            return ("a", int(batch.shape[0]), simulator)

    class B:
        def train_step(self, simulator, batch):
            return ("b", int(batch.shape[0]), simulator)

    assert p.train_step(runtime=A()) == ("a", 4, sim)
    assert p.train_step(runtime=B()) == ("b", 4, sim)
    magat, gpt = Recorder("magat"), Recorder("mapf_gpt")
    assert p.train_step(runtime=magat) == {"backend": "magat", "rows": 4}
    assert p.train_step(runtime=gpt) == {"backend": "mapf_gpt", "rows": 4}
    assert magat.calls[0][0] is sim and gpt.calls[0][0] is sim


@pytest.mark.parametrize("backend", ["magat", "mapf_gpt"])
def test_each_frontier_is_filtered_on_its_own_reset_rows(backend):
    p = pipeline_for(two_env_sim())
    first = frontier(reset=(1, 0, 0, 1), actions=(4, 0, 1, 3))
    second = frontier(reset=(0, 1, 0, 0), positions=((10, 11), (10, 11), (19, 20), (20, 20)), actions=(0, 4, 0, 4))
    subsets = [first[[0, 3]], second[[1]]]
    mocked_stage(p, first, second, reset_subsets=subsets)
    rt = Recorder(backend)
    assert p.train_step(runtime=rt)["rows"] == p.train_step(runtime=rt)["rows"] == 4
    filtered = [c.args[0] for c in p.gpu_handler.filter_reset_agents.call_args_list]
    processed = [c.args for c in p.gpu_handler.process_batch.call_args_list]
    assert len(filtered) == len(processed) == len(rt.calls) == 2
    for k, (stage, subset) in enumerate(((first, subsets[0]), (second, subsets[1]))):
        assert torch.equal(filtered[k], stage) and torch.equal(rt.calls[k][1], stage)
        assert torch.equal(processed[k][0], stage) and torch.equal(processed[k][1], subset)
    assert subsets[0][:, 0].tolist() == [0, 1] and subsets[1][:, 0].tolist() == [0]


# ---- two frontiers through the real ring and DMA worker -------------------------------------------
FIRST = dict(reset=(1, 0, 0, 1), positions=((10, 10), (10, 11), (20, 20), (20, 21)), actions=(4, 0, 1, 3))
SECOND = dict(reset=(0, 1, 1, 0), positions=((30, 30), (30, 31), (40, 40), (40, 41)), actions=(0, 4, 4, 0))


def written_pipeline():
    p = pipeline_for(two_env_sim())
    first, second = frontier(**FIRST), frontier(**SECOND)
    for f in (first, second):
        for block in env_blocks(f):
            p.ring_buffer.reserve_and_write(block)
    return p, first, second


@pytest.mark.parametrize("backend", ["magat", "mapf_gpt"])
def test_counters_after_each_frontier(backend):
    p, first, second = written_pipeline()
    p.gpu_handler = MagicMock()
    p.gpu_handler.filter_reset_agents.side_effect = lambda b: b[b[:, RESET_FLAG_COL] != 0]
    assert p.has_env_aligned_batch(2) is True
    rt = Recorder(backend)
    with cpu_device():
        assert p.dma_worker.run_once() == (0, 4)
        s = p.get_stats()
        assert (s["dma_read_ptr"], s["compute_ptr"], s["reserve_ptr"]) == (4, 0, 8)
        assert s["stage_ready_counts"] == [2, 2] and s["stage_seq_tags"] == [0, 1]
        assert p.train_step(runtime=rt)["rows"] == 4
        s = p.get_stats()
        assert (s["compute_ptr"], s["dma_read_ptr"]) == (4, 4)
        assert s["stage_ready_counts"] == [0, 2] and s["stage_seq_tags"] == [-1, 1]
        assert s["env_write_stage"] == [2, 2]
        assert p.has_env_aligned_batch(2) is True
        assert p.extract_env_aligned_batch(4, agents_per_env=2, num_envs=2) is None  # not uploaded yet
        assert p.dma_worker.run_once() == (4, 8)
        s = p.get_stats()
        assert (s["dma_read_ptr"], s["compute_ptr"]) == (8, 4)
        assert p.train_step(runtime=rt)["rows"] == 4
    s = p.get_stats()
    assert (s["compute_ptr"], s["dma_read_ptr"], s["reserve_ptr"]) == (8, 8, 8)
    assert s["stage_ready_counts"] == [0, 0] and s["stage_seq_tags"] == [-1, -1]
    assert s["env_write_stage"] == [2, 2]
    assert p.has_env_aligned_batch(2) is False
    assert torch.equal(rt.calls[0][1], first) and torch.equal(rt.calls[1][1], second)


@pytest.mark.parametrize("backend", ["magat", "mapf_gpt"])
def test_backend_sees_frontier_local_stages_and_post_release_stats(backend):
    p, first, second = written_pipeline()
    p.gpu_handler = MagicMock()
    p.gpu_handler.filter_reset_agents.side_effect = lambda b: b[b[:, RESET_FLAG_COL] != 0]
    seen = []

    def observe(rt, stage):
        seen.append({"stats": p.get_stats(), "ready": p.has_env_aligned_batch(2)})
        return {"call_index": len(rt.calls) - 1, "reset_rows": int((stage[:, RESET_FLAG_COL] != 0).sum()),
                "env_ids": stage[:, 0].tolist(), "positions": stage[:, 2:4].tolist()}

    rt = Recorder(backend, extra=observe)
    with cpu_device():
        assert p.dma_worker.run_once() == (0, 4)
        r0 = p.train_step(runtime=rt)
        assert p.dma_worker.run_once() == (4, 8)
        r1 = p.train_step(runtime=rt)
    assert r0 == {"backend": backend, "rows": 4, "call_index": 0, "reset_rows": 2, "env_ids": [0, 0, 1, 1],
                  "positions": [[10, 10], [10, 11], [20, 20], [20, 21]]}
    assert r1 == {"backend": backend, "rows": 4, "call_index": 1, "reset_rows": 2, "env_ids": [0, 0, 1, 1],
                  "positions": [[30, 30], [30, 31], [40, 40], [40, 41]]}
    base = {"capacity": 8, "reserve_ptr": 8, "num_stage_slots": 2, "stage_rows": 4, "env_write_stage": [2, 2]}
    assert seen[0] == {"stats": {**base, "dma_read_ptr": 4, "compute_ptr": 4, "stage_ready_counts": [0, 2],
                                 "stage_seq_tags": [-1, 1]}, "ready": True}
    assert seen[1] == {"stats": {**base, "dma_read_ptr": 8, "compute_ptr": 8, "stage_ready_counts": [0, 0],
                                 "stage_seq_tags": [-1, -1]}, "ready": False}


@pytest.mark.parametrize("backend", ["magat", "mapf_gpt"])
def test_failure_on_the_second_frontier_leaves_it_consumed(backend):
    p, first, second = written_pipeline()
    p.gpu_handler = MagicMock()
    p.gpu_handler.filter_reset_agents.side_effect = lambda b: b[:0]
    aggregate = []

    def keep(rt, stage):
        aggregate.append(stage[:, 2:4].tolist())
        return {"aggregate": [list(a) for a in aggregate]}

    rt = Recorder(backend, fail_on=2, extra=keep)
    with cpu_device():
        assert p.dma_worker.run_once() == (0, 4)
        first_result = p.train_step(runtime=rt)
        assert p.dma_worker.run_once() == (4, 8)
        with pytest.raises(RuntimeError, match=f"{backend} frontier failure"):
            p.train_step(runtime=rt)
    assert first_result["aggregate"] == [[[10, 10], [10, 11], [20, 20], [20, 21]]]
    assert aggregate == first_result["aggregate"]  # the failed call added nothing
    s = p.get_stats()
    assert (s["compute_ptr"], s["dma_read_ptr"], s["reserve_ptr"]) == (8, 8, 8)
    assert s["stage_ready_counts"] == [0, 0] and s["stage_seq_tags"] == [-1, -1]
    assert s["env_write_stage"] == [2, 2]
    assert p.has_env_aligned_batch(2) is False
    assert len(rt.calls) == 2 and torch.equal(rt.calls[0][1], first) and torch.equal(rt.calls[1][1], second)
