"""CPU tests of the expert-record ring (iclr_2027_jointoom_amd/ring.py).

Ports /root/reference/tests/expert/test_ring_fail_stop.py and the
RingBuffer / DMAWorker cases of tests/expert/test_pipeline.py:170-320, and
adds the stage protocol, the staged DMA data path (device calls replaced by
mocks, as the reference's fail-stop test does), frozen-record round trips
and record producers started from a forkserver (their shutdown included).
"""
import contextlib
import multiprocessing as mp
import os
import threading
import time
from unittest.mock import MagicMock, patch

import numpy as np
import pytest
import torch

from iclr_2027_jointoom_amd.ring import (
    FEATURE_DIM,
    MAPFGPT_FEATURE_DIM,
    DMAWorker,
    RingBuffer,
    RingStageSource,
    load_records,
    save_records,
    validate_stage,
)

_HARD_EXIT_CODE = 73


@contextlib.contextmanager
def cpu_device():
    """Run DMAWorker's device calls on the CPU (pinning, streams, events)."""
    with patch("torch.Tensor.pin_memory", lambda self: self), \
            patch("torch.cuda.Stream", return_value=object()), \
            patch("torch.cuda.Event", side_effect=lambda **kw: MagicMock()), \
            patch("torch.cuda.stream", lambda s: contextlib.nullcontext()):
        yield


def env_block(env_id, agents=2, features=FEATURE_DIM, fill=0):
    block = np.zeros((agents, features), dtype=np.uint16)
    block[:, 0] = env_id
    block[:, 1] = np.arange(agents, dtype=np.uint16)
    block[:, 2:] = fill
    return block


# ---- RingBuffer (test_pipeline.py:170-265) ------------------------------------------------------
def test_init_sizes_and_shared_memory():
    buf = RingBuffer(capacity=1024, feature_dim=FEATURE_DIM)
    assert buf.capacity == 1024 and buf.feature_dim == FEATURE_DIM
    assert buf.cpu_buffer.shape == (1024, FEATURE_DIM) and buf.cpu_buffer.dtype == torch.int16
    assert len(buf.ready_flags) == 1024 and not buf.cpu_buffer.is_cuda
    assert buf.cpu_buffer.is_shared() and buf.shared_reserve_ptr.value == 0


def test_reserve_and_write_wraps_and_scans():
    buf = RingBuffer(capacity=64)
    data = np.zeros((10, FEATURE_DIM), dtype=np.uint16)
    data[:, 0], data[:, 6] = 1, 2
    assert buf.reserve_and_write(data) == (0, 10) and buf.shared_reserve_ptr.value == 10
    assert buf.scan_ready_range(0, 20) == 10
    buf.clear_flags(0, 10)
    assert sum(buf.ready_flags[:10]) == 0
    buf.shared_compute_ptr.value = 60
    buf.shared_reserve_ptr.value = 60
    data2 = np.arange(10 * FEATURE_DIM, dtype=np.uint16).reshape(10, FEATURE_DIM)
    assert buf.reserve_and_write(data2) == (60, 6)  # wraps: 4 rows at the end, 6 at the start
    assert np.array_equal(buf.cpu_buffer[60:64].numpy(), data2[:4].astype(np.int16))
    assert np.array_equal(buf.cpu_buffer[0:6].numpy(), data2[4:].astype(np.int16))
    with pytest.raises(ValueError, match="cannot write chunk"):
        buf.reserve_and_write(np.zeros((65, FEATURE_DIM), np.uint16))


def test_multiprocess_shared_access():
    buf = RingBuffer(capacity=64)
    p = mp.get_context("fork").Process(target=lambda: setattr(buf.shared_reserve_ptr, "value", 42))
    p.start()
    p.join(timeout=5)
    assert buf.shared_reserve_ptr.value == 42


def test_reserve_blocks_when_unconsumed_window_is_full():
    buf = RingBuffer(capacity=16)
    data = np.zeros((8, FEATURE_DIM), dtype=np.uint16)
    buf.reserve_and_write(data)
    buf.reserve_and_write(data)
    done = {"v": False}

    def writer():
        buf.reserve_and_write(data)
        done["v"] = True

    t = threading.Thread(target=writer, daemon=True)
    t.start()
    time.sleep(0.05)
    assert t.is_alive() and not done["v"]
    buf.clear_flags(0, 8)
    buf.shared_compute_ptr.value = 8
    t.join(timeout=1.0)
    assert done["v"] and not t.is_alive()


# ---- stage protocol ----------------------------------------------------------------------------
def test_stage_layout_validation():
    with pytest.raises(ValueError, match="divisible"):
        RingBuffer(capacity=10, num_envs=2, agents_per_env=3)
    with pytest.raises(ValueError, match="num_envs must be positive"):
        RingBuffer(capacity=8, num_envs=0, agents_per_env=2)
    ring = RingBuffer(capacity=8, num_envs=2, agents_per_env=2)
    assert ring.stage_mode and ring.stage_rows == 4 and ring.num_stage_slots == 2
    with pytest.raises(ValueError, match="one full env block"):
        ring.reserve_and_write(env_block(0, agents=3))
    with pytest.raises(ValueError, match="env_id out of range"):
        ring.reserve_and_write(env_block(2))
    bad = env_block(0)
    bad[1, 0] = 1
    with pytest.raises(ValueError, match="single env_id"):
        ring.reserve_and_write(bad)
    bad = env_block(0)
    bad[:, 1] = [1, 0]
    with pytest.raises(ValueError, match="contiguous"):
        ring.reserve_and_write(bad)


def test_stage_visible_only_when_every_env_published_and_slots_recycle():
    ring = RingBuffer(capacity=8, num_envs=2, agents_per_env=2)
    ring.reserve_and_write(env_block(0, fill=1))
    assert not ring.is_stage_ready(0)
    ring.reserve_and_write(env_block(1, fill=2))
    assert ring.is_stage_ready(0)
    # env 0 runs ahead into stage 1 (slot 1), then must wait for slot 0 to be released
    ring.reserve_and_write(env_block(0, fill=3))
    done = {"v": False}

    def third():
        ring.reserve_and_write(env_block(0, fill=5))  # stage 2 -> slot 0, still unconsumed
        done["v"] = True

    t = threading.Thread(target=third, daemon=True)
    t.start()
    time.sleep(0.05)
    assert not done["v"]
    ring.release_stage(0)
    ring.shared_compute_ptr.value = ring.stage_rows
    t.join(timeout=1.0)
    assert done["v"]
    assert ring.stage_seq_tags[0] == 2 and not ring.is_stage_ready(2)
    assert list(ring.env_write_seq) == [3, 1]


def _reserve_then_hard_exit(ring, reserved):
    ring._reserve_stage_block(env_id=0)
    reserved.set()
    os._exit(_HARD_EXIT_CODE)


def test_hard_exit_after_reserve_keeps_partial_stage_invisible_and_restartable():
    """test_ring_fail_stop.py:40-79."""
    ctx = mp.get_context("fork")
    ring = RingBuffer(capacity=8, num_envs=2, agents_per_env=2)
    reserved = ctx.Event()
    child = ctx.Process(target=_reserve_then_hard_exit, args=(ring, reserved))
    started = time.monotonic()
    child.start()
    assert reserved.wait(timeout=2.0)
    child.join(timeout=2.0)
    assert not child.is_alive() and child.exitcode == _HARD_EXIT_CODE
    assert time.monotonic() - started < 2.0
    assert ring.stage_seq_tags[0] == 0 and ring.stage_ready_counts[0] == 0
    assert list(ring.env_write_seq) == [0, 0] and sum(ring.ready_flags[:4]) == 0
    assert ring.is_stage_ready(0) is False
    with cpu_device():
        dma = DMAWorker(ring, torch.zeros((8, FEATURE_DIM), dtype=torch.int16), batch_threshold=4, device="cpu")
    assert dma.run_once() is None and dma.dma_read_ptr == 0
    fresh = RingBuffer(capacity=8, num_envs=2, agents_per_env=2)
    fresh.reserve_and_write(env_block(0))
    fresh.reserve_and_write(env_block(1))
    assert fresh.is_stage_ready(0) is True


# ---- DMAWorker ------------------------------------------------------------------------------------
def test_dma_worker_interface():
    """test_pipeline.py:266-320."""
    ring = RingBuffer(capacity=1024)
    with cpu_device():
        w = DMAWorker(ring, torch.zeros((1024, FEATURE_DIM), dtype=torch.int16), batch_threshold=256)
        assert w.batch_threshold == 256 and w.dma_read_ptr == 0
        assert w.run_once() is None
        assert w.gpu_buffer.shape == ring.cpu_buffer.shape
        t = w.start()
        assert isinstance(t, threading.Thread)
        w.stop()
        assert w._running is False


def test_dma_moves_stages_through_staging_slots_in_order():
    ring = RingBuffer(capacity=12, num_envs=2, agents_per_env=2)  # 3 stage slots
    with cpu_device():
        gpu = torch.zeros((12, FEATURE_DIM), dtype=torch.int16)
        dma = DMAWorker(ring, gpu, device="cpu", staging_slots=2)
    for stage in range(5):
        for env in range(2):
            ring.reserve_and_write(env_block(env, fill=10 * stage + env + 1))
        with cpu_device():
            assert dma.run_once() == ring._stage_row_bounds(stage)
        lo, hi = ring._stage_row_bounds(stage)
        assert np.array_equal(gpu[lo:hi, 2].numpy(), [10 * stage + 1] * 2 + [10 * stage + 2] * 2)
        with cpu_device():
            assert dma.run_once() is None  # next stage not published yet
        dma.release_completed_stage(stage)
        assert ring.shared_compute_ptr.value == (stage + 1) * 4
    assert dma.dma_read_ptr == 20


def test_dma_non_stage_mode_copies_ready_rows():
    ring = RingBuffer(capacity=64)
    with cpu_device():
        gpu = torch.zeros((64, FEATURE_DIM), dtype=torch.int16)
        dma = DMAWorker(ring, gpu, device="cpu")
    data = np.arange(10 * FEATURE_DIM, dtype=np.uint16).reshape(10, FEATURE_DIM)
    ring.reserve_and_write(data)
    with cpu_device():
        assert dma.run_once() == (0, 10)
    assert np.array_equal(gpu[:10].numpy(), data.astype(np.int16))
    assert sum(ring.ready_flags[:10]) == 0 and dma.dma_read_ptr == 10


# ---- frozen records ---------------------------------------------------------------------------------
def make_records(E=2, A=3, S=4, W=8, features=MAPFGPT_FEATURE_DIM, seed=0):
    rng = np.random.default_rng(seed)
    grids = np.zeros((E, W, W), np.uint8)
    grids[:, 0, 0] = 1
    stages = np.zeros((S, E * A, features), np.uint16)
    for s in range(S):
        blk = stages[s].reshape(E, A, features)
        blk[:, :, 0] = np.arange(E)[:, None]
        blk[:, :, 1] = np.arange(A)[None]
        for e in range(E):
            cells = rng.choice(np.arange(1, W * W), size=2 * A, replace=False)
            blk[e, :, 2], blk[e, :, 3] = cells[:A] // W, cells[:A] % W
            blk[e, :, 4], blk[e, :, 5] = cells[A:] // W, cells[A:] % W
        blk[:, :, 6] = rng.integers(0, 5, size=(E, A))
        blk[:, :, 7] = s == 0
        if features > FEATURE_DIM:
            blk[:, :, 8:] = 5
    return grids, stages


def test_validate_stage_rejections():
    grids, stages = make_records(features=FEATURE_DIM)
    validate_stage(stages[0], grids, 3, FEATURE_DIM)
    cases = {
        "environment-major": lambda s: s.astype(np.int32),
        "environment order": lambda s: s.__setitem__((0, 0), 1),
        "agent order": lambda s: s.__setitem__((0, 1), 2),
        "invalid action": lambda s: s.__setitem__((0, 6), 5),
        "outside map": lambda s: s.__setitem__((0, 2), 8),
        "on obstacles": lambda s: (s.__setitem__((0, 2), 0), s.__setitem__((0, 3), 0)),
        "duplicate": lambda s: (s.__setitem__((1, 2), s[0, 2]), s.__setitem__((1, 3), s[0, 3])),
    }
    for msg, mutate in cases.items():
        s = stages[0].copy()
        out = mutate(s)
        s = out if isinstance(out, np.ndarray) else s
        with pytest.raises(ValueError, match=msg):
            validate_stage(s, grids, 3, FEATURE_DIM)


def test_save_load_round_trip_and_hash_check(tmp_path):
    grids, stages = make_records()
    m = save_records(tmp_path / "rec", backend="mapf_gpt", grids=grids, stages=stages, metadata={"seed": 0})
    assert m["features"] == 13 and m["agents"] == 3 and m["stages"] == 4
    m2, g2, s2 = load_records(tmp_path / "rec")
    assert m2 == m and np.array_equal(g2, grids) and np.array_equal(s2, stages)
    assert isinstance(s2, np.memmap)
    with pytest.raises(FileExistsError):
        save_records(tmp_path / "rec", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    raw = bytearray((tmp_path / "rec" / "stages.npy").read_bytes())
    raw[-1] ^= 1
    (tmp_path / "rec" / "stages.npy").write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="hash mismatch"):
        load_records(tmp_path / "rec")


def test_ring_stage_source_streams_frozen_records_in_order(tmp_path):
    grids, stages = make_records(E=3, A=4, S=6)
    save_records(tmp_path / "rec", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    ring = RingBuffer(capacity=2 * 12, feature_dim=13, num_envs=3, agents_per_env=4)
    config = {"num_agents": 4, "num_steps": 6, "map_names": ["a", "b", "c"]}
    src = RingStageSource(ring, "mapf_gpt", config, records=tmp_path / "rec", timeout=20)
    try:
        src.start()
        for s in range(6):
            assert np.array_equal(src.next_rows(), stages[s]), s
        with pytest.raises(StopIteration):
            src.next_rows()
    finally:
        src.close()


def test_producers_are_spawned_where_signal_handlers_are_foreign(tmp_path, monkeypatch):
    """A SIGCHLD handler installed outside Python (as a preloaded profiler
    library installs one) makes the forkserver's children exit at once, so
    the producers are spawned instead, and they stream the same stages."""
    from iclr_2027_jointoom_amd import ring as ring_mod

    real = ring_mod.signal.getsignal
    monkeypatch.setattr(ring_mod.signal, "getsignal",
                        lambda s: None if s == ring_mod.signal.SIGCHLD else real(s))
    monkeypatch.setattr(ring_mod, "_CONTEXT", None)
    assert ring_mod._process_context().get_start_method() == "spawn"
    grids, stages = make_records(E=2, A=3, S=4)
    save_records(tmp_path / "rec", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    ring = RingBuffer(capacity=2 * 6, feature_dim=13, num_envs=2, agents_per_env=3)
    config = {"num_agents": 3, "num_steps": 4, "map_names": ["a", "b"]}
    src = RingStageSource(ring, "mapf_gpt", config, records=tmp_path / "rec", timeout=60, workers=2)
    try:
        src.start()
        for s in range(4):
            assert np.array_equal(src.next_rows(), stages[s]), s
    finally:
        src.close()


def test_close_stops_blocked_producers_without_terminating_them(tmp_path):
    """Producers waiting for a free slot (the consumer stopped reading) exit
    by themselves when the source closes: exit code 0, no SIGTERM, well
    within the grace period.  They are forkserver children, not forks of
    the consumer."""
    grids, stages = make_records(E=3, A=4, S=8)
    save_records(tmp_path / "rec", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    ring = RingBuffer(capacity=12, feature_dim=13, num_envs=3, agents_per_env=4)  # one stage slot
    config = {"num_agents": 4, "num_steps": 8, "map_names": ["a", "b", "c"]}
    src = RingStageSource(ring, "mapf_gpt", config, records=tmp_path / "rec", timeout=20, workers=2)
    assert all(p._start_method == "forkserver" for p in src.processes)
    src.start()
    assert np.array_equal(src.next_rows(), stages[0])
    time.sleep(0.2)  # the producers now wait for the slot of stage 2
    assert all(p.is_alive() for p in src.processes)
    started = time.monotonic()
    src.close()
    assert time.monotonic() - started < 3.0
    assert [p.exitcode for p in src.processes] == [0, 0]


def test_finished_producers_exit_and_a_failing_one_is_reported(tmp_path):
    grids, stages = make_records(E=2, A=4, S=3)
    save_records(tmp_path / "rec", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    ring = RingBuffer(capacity=3 * 8, feature_dim=13, num_envs=2, agents_per_env=4)
    src = RingStageSource(ring, "mapf_gpt", {"num_agents": 4, "num_steps": 3, "map_names": ["a", "b"]},
                          records=tmp_path / "rec", timeout=20)
    try:
        src.start()
        for p in src.processes:
            p.join(10)
        assert [p.exitcode for p in src.processes] == [0, 0]
        src.check()  # finished producers are not failures
        assert [np.array_equal(src.next_rows(), stages[s]) for s in range(3)] == [True] * 3
    finally:
        src.close()
    # blocks of 3 rows into a ring of 4 agents per env: the producers raise
    ring = RingBuffer(capacity=8, feature_dim=13, num_envs=2, agents_per_env=4)
    src = RingStageSource(ring, "mapf_gpt", {"num_agents": 3, "num_steps": 3, "map_names": ["a", "b"]},
                          records=tmp_path / "rec", timeout=20)
    try:
        src.start()
        for p in src.processes:
            p.join(10)
        with pytest.raises(RuntimeError, match="expert process exited"):
            src.check()
    finally:
        src.close()


def test_ring_stage_source_without_records_is_not_built():
    ring = RingBuffer(capacity=8, num_envs=2, agents_per_env=2)
    with pytest.raises(NotImplementedError, match="live expert producers"):
        RingStageSource(ring, "magat", {"num_agents": 2, "num_steps": 1, "map_names": ["a", "b"]})


def test_stage_ready_counts_and_reserve_pointer_follow_the_env_words():
    ring = RingBuffer(capacity=8, num_envs=2, agents_per_env=2)
    assert list(ring.stage_ready_counts) == [0, 0] and ring.shared_reserve_ptr.value == 0
    ring.reserve_and_write(env_block(1, fill=4))
    assert list(ring.stage_ready_counts) == [1, 0] and ring.shared_reserve_ptr.value == 2
    ring.write_stage_range(0, np.concatenate([env_block(0, fill=1)]))
    assert list(ring.stage_ready_counts) == [2, 0] and ring.is_stage_ready(0)
    # one producer writing both envs of the next stage with one reservation
    both = np.concatenate([env_block(0, fill=7), env_block(1, fill=8)])
    assert ring.write_stage_range(0, both) == ring._stage_row_bounds(1)
    assert ring.is_stage_ready(1) and list(ring.env_write_seq) == [2, 2]
    assert np.array_equal(ring.cpu_buffer[4:8, 2].numpy(), [7, 7, 8, 8])
    with pytest.raises(ValueError, match="single env_id"):
        ring.write_stage_range(0, np.concatenate([env_block(1), env_block(0)]))
    ring.release_stage(0)
    assert list(ring.stage_ready_counts) == [0, 2] and not ring.is_stage_ready(0)


def test_stage_ring_requires_total_store_order():
    """Stage publication is lock-free and fence-free: hosts without x86-64's
    store order are refused up front rather than left to race."""
    from iclr_2027_jointoom_amd.ring import _require_total_store_order

    _require_total_store_order("x86_64")
    _require_total_store_order("AMD64")
    for machine in ("aarch64", "ppc64le", "riscv64"):
        with pytest.raises(RuntimeError, match="total store order"):
            _require_total_store_order(machine)
    with patch("platform.machine", return_value="aarch64"):
        with pytest.raises(RuntimeError, match="total store order"):
            RingBuffer(capacity=8, num_envs=2, agents_per_env=2)
        RingBuffer(capacity=8)  # the stage-less ring takes reserve_lock
