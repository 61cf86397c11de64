"""CPU tests of the compact expert-record format (iclr_2027_jointoom_amd/records.py),
its ring (CompactRingBuffer) and the oracle that restates the producers' rows
(oracle/records.py).

The oracle is pinned by the reference's known answers for the history rule
(test_mapf_gpt_schema.py:12-28, test_mapf_gpt_online.py:19-45) and the row
layouts (test_mapf_gpt_schema.py:31-55, test_pipeline.py:558-574)."""
import json

import numpy as np
import pytest
import torch

from iclr_2027_jointoom_amd.records import (
    CompactRecords,
    compact_from_stages,
    load_compact_records,
    save_compact_records,
    write_compact_records,
)
from iclr_2027_jointoom_amd.ring import (
    CompactRingBuffer,
    RingBuffer,
    RingStageSource,
    load_records,
    save_records,
)
from oracle.records import History, expand_records
from records_data import make_compact


# ---- oracle pins ------------------------------------------------------------------------------
def test_history_kat_snapshots_previous_five_actions_and_resets():
    """test_mapf_gpt_schema.py:12-28, through the stage expansion."""
    acts = [0, 1, 2, 3, 4, 0]
    S = len(acts) + 1
    positions = np.zeros((S, 1, 2), np.uint16)
    actions = np.array(acts + [2], np.uint8).reshape(S, 1)
    starts = np.zeros((S, 1), np.uint8)
    starts[0] = starts[S - 1] = 1  # the last stage opens a new episode: reset
    goals = np.zeros((2, 1, 2), np.uint16)
    rows = expand_records(positions, actions, starts, goals, 1, 13)
    snaps = [rows[s, 0, 8:13].tolist() for s in range(S)]
    assert snaps[0] == [5, 5, 5, 5, 5]
    assert snaps[1] == [5, 5, 5, 5, 0]
    assert snaps[5] == [0, 1, 2, 3, 4]
    assert snaps[6] == [5, 5, 5, 5, 5]  # reset
    h = History(1)
    h.append([0]); h.append([1]); h.append([2]); h.append([3]); h.append([4]); h.append([0])
    assert h.snapshot() == [[1, 2, 3, 4, 0]]


def test_step_builder_kat_history_before_current_action():
    """test_mapf_gpt_online.py:19-45 (env 1 of 2, two agents, offset 5 removed)."""
    positions = np.zeros((3, 4, 2), np.uint16)
    goals = np.zeros((2, 2, 2), np.uint16)
    for a in range(2):
        positions[:, 2 + a] = (10, 11 + a)
        positions[:, a] = (0, a)
        goals[:, a] = (20, 21 + a)
    actions = np.zeros((3, 4), np.uint8)
    actions[0, 2:] = (1, 4)
    actions[1, 2:] = (2, 3)
    actions[2, 2:] = (2, 3)
    starts = np.array([[1, 1], [0, 0], [0, 1]], np.uint8)
    # goal blocks in (stage, env) order: (0,0), (0,1), (2,1)
    goal_blocks = np.stack([goals[0] * 0, goals[0], goals[0]])
    rows = expand_records(positions, actions, starts, goal_blocks, 2, 13)
    t0, t1, t2 = rows[0, 2:], rows[1, 2:], rows[2, 2:]
    assert np.all(t0[:, 0] == 1) and np.array_equal(t0[:, 1], [0, 1])
    assert np.all(t0[:, 8:13] == 5) and np.array_equal(t0[:, 6], [1, 4])
    assert t0[:, 2:6].tolist() == [[10, 11, 20, 21], [10, 12, 20, 22]]
    assert np.array_equal(t1[:, 8:13], [[5, 5, 5, 5, 1], [5, 5, 5, 5, 4]])
    assert not np.any(t1[:, 8:13] == t1[:, 6:7])
    assert np.all(t2[:, 8:13] == 5) and np.all(t2[:, 7] == 1)


def test_row_layout_kats():
    """Column order of test_mapf_gpt_schema.py:31-55 (per-env flag variant)
    and test_pipeline.py:558-574 (8 columns, env 3)."""
    positions = np.array([[[5, 6], [7, 8]]], np.uint16)
    rows = expand_records(positions, np.array([[3, 4]], np.uint8), np.array([[1]], np.uint8),
                          np.array([[[9, 10], [11, 12]]], np.uint16), 1, 13)
    assert rows[0, :, :8].tolist() == [[0, 0, 5, 6, 9, 10, 3, 1], [0, 1, 7, 8, 11, 12, 4, 1]]
    E, A = 4, 4
    positions = np.zeros((1, E * A, 2), np.uint16)
    positions[0, 3 * A:] = (5, 15)
    goals = np.zeros((E, A, 2), np.uint16)
    goals[3] = (45, 55)
    rows = expand_records(positions, np.tile(np.array([1, 2, 3, 4], np.uint8), E)[None], np.ones((1, E), np.uint8),
                          goals, E, 8)
    blk = rows[0, 3 * A:]
    assert rows.shape == (1, E * A, 8)
    assert np.all(blk[:, 0] == 3) and np.array_equal(blk[:, 1], [0, 1, 2, 3])
    assert np.all(blk[:, 2] == 5) and np.all(blk[:, 3] == 15)
    assert np.all(blk[:, 4] == 45) and np.all(blk[:, 5] == 55) and np.all(blk[:, 7] == 1)


# ---- encoder ----------------------------------------------------------------------------------
@pytest.mark.parametrize("features", [8, 13])
def test_compact_round_trip_equals_inputs(features):
    E, A, S = 3, 5, 30
    grids, arrays = make_compact(3, E, 16, A, S)
    stages = expand_records(*arrays, E, features)
    rec = compact_from_stages(stages, E, features)
    for got, want in zip((rec.positions, rec.actions, rec.episode_starts, rec.goals), arrays):
        assert got.dtype == want.dtype and np.array_equal(got, want)
    assert rec.agents == A and rec.num_envs == E and rec.num_stages == S
    assert np.array_equal(expand_records(rec.positions, rec.actions, rec.episode_starts, rec.goals, E, features),
                          stages)


def test_encoder_rejects_rows_the_producers_do_not_write():
    E, A, S = 2, 4, 8
    _, arrays = make_compact(5, E, 16, A, S)
    stages = expand_records(*arrays, E, 13)
    later = int(np.flatnonzero(arrays[2][:, 0] == 0)[1])  # a stage that continues env 0's episode
    cases = {
        "one refresh flag per env": lambda s: s.__setitem__((later, 0, 7), 1),
        "start an episode at stage 0": lambda s: s.__setitem__((0, slice(0, A), 7), 0),
        "change only at an episode start": lambda s: s.__setitem__((later, 1, 4), s[later, 1, 4] + 1),
        "previous actions": lambda s: s.__setitem__((later, 2, 12), (s[later, 2, 12] + 1) % 5),
        "agent order": lambda s: s.__setitem__((1, 0, 1), 3),
        "invalid action": lambda s: s.__setitem__((1, 0, 6), 5),
    }
    for msg, mutate in cases.items():
        s = stages.copy()
        mutate(s)
        with pytest.raises(ValueError, match=msg):
            compact_from_stages(s, E, 13)


def test_compact_archive_round_trip_hash_and_validation(tmp_path):
    E, A, S = 3, 6, 12
    grids, arrays = make_compact(11, E, 16, A, S)
    stages = expand_records(*arrays, E, 13)
    m = save_compact_records(tmp_path / "c", backend="mapf_gpt", grids=grids, stages=stages, metadata={"s": 1})
    assert m["format"] == "compact" and m["features"] == 13 and m["agents"] == A and m["stages"] == S
    # 5 bytes per agent and step (plus goal blocks and one flag byte per env and stage)
    assert (tmp_path / "c" / "positions.npy").stat().st_size < S * E * A * 4 + 256
    m2, g2, rec = load_compact_records(tmp_path / "c")
    assert m2 == m and np.array_equal(g2, grids)
    assert isinstance(rec.positions, np.memmap)
    assert np.array_equal(expand_records(rec.positions, rec.actions, rec.episode_starts, rec.goals, E, 13), stages)
    with pytest.raises(FileExistsError):
        save_compact_records(tmp_path / "c", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    raw = bytearray((tmp_path / "c" / "actions.npy").read_bytes())
    raw[-1] ^= 1
    (tmp_path / "c" / "actions.npy").write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="hash mismatch"):
        load_compact_records(tmp_path / "c")
    # the full-row loader refuses a compact manifest and vice versa
    with pytest.raises(ValueError, match="unsupported"):
        load_records(tmp_path / "c")
    save_records(tmp_path / "full", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    with pytest.raises(ValueError, match="unsupported"):
        load_compact_records(tmp_path / "full")


def test_compact_validation_matches_validate_stage_rules(tmp_path):
    E, A, S = 2, 4, 3
    grids, arrays = make_compact(2, E, 16, A, S)
    obstacle = np.argwhere(grids[0] != 0)[0]
    cases = {
        "outside map": lambda p, a, st, g: p.__setitem__((1, 0, 0), 16),
        "on obstacles": lambda p, a, st, g: p.__setitem__((1, 0), obstacle),
        "duplicate": lambda p, a, st, g: p.__setitem__((1, 1), p[1, 0]),
        "invalid action": lambda p, a, st, g: a.__setitem__((2, 3), 7),
    }
    for i, (msg, mutate) in enumerate(cases.items()):
        p, a, st, g = (x.copy() for x in arrays)
        mutate(p, a, st, g)
        rec = CompactRecords(p, a, st, g)
        with pytest.raises(ValueError, match=msg):
            write_compact_records(tmp_path / f"bad{i}", backend="mapf_gpt", grids=grids, records=rec, metadata={})
    p, a, st, g = (x.copy() for x in arrays)
    g[0, 1] = g[0, 0]
    with pytest.raises(ValueError, match="duplicate"):
        write_compact_records(tmp_path / "badg", backend="magat", grids=grids, records=CompactRecords(p, a, st, g),
                              metadata={})


# ---- compact ring ------------------------------------------------------------------------------
def _decode_slot(ring: CompactRingBuffer, seq: int):
    slot = ring.slot_view(seq)
    N, E = ring.stage_rows, ring.num_envs
    pos = slot[:4 * N].view(np.uint16).reshape(N, 2)
    act = slot[ring.off_actions:ring.off_actions + N]
    st = slot[ring.off_starts:ring.off_starts + E]
    goals = slot[ring.off_goals:ring.off_goals + 4 * N].view(np.uint16).reshape(E, -1, 2)
    return pos.copy(), act.copy(), st.copy(), goals.copy()


def test_compact_ring_layout_and_stage_protocol():
    E, A = 3, 4
    ring = CompactRingBuffer(2 * E * A, 13, num_envs=E, agents_per_env=A)
    assert ring.cpu_buffer.dtype == torch.uint8 and ring.cpu_buffer.shape == (2, ring.slot_bytes)
    assert ring.off_goals % 16 == 0 and ring.slot_bytes % 64 == 0 and ring.head_bytes == 5 * E * A + E
    rng = np.random.default_rng(0)
    pos = rng.integers(0, 100, size=(E * A, 2)).astype(np.uint16)
    act = rng.integers(0, 5, size=E * A).astype(np.uint8)
    goals = rng.integers(0, 100, size=(E * A, 2)).astype(np.uint16)
    ring.write_compact(0, pos[:2 * A], act[:2 * A], [1, 0], goals[:2 * A])
    assert not ring.is_stage_ready(0)
    ring.write_compact(2, pos[2 * A:], act[2 * A:], [1], goals[2 * A:])
    assert ring.is_stage_ready(0) and list(ring.env_write_seq) == [1, 1, 1]
    p, a, st, g = _decode_slot(ring, 0)
    assert np.array_equal(p, pos) and np.array_equal(a, act) and st.tolist() == [1, 0, 1]
    assert np.array_equal(g[0], goals[:A]) and np.array_equal(g[2], goals[2 * A:])
    assert ring.shared_reserve_ptr.value == E * A and sum(ring.ready_flags[:E * A]) == E * A
    ring.release_stage(0)
    assert sum(ring.ready_flags[:E * A]) == 0
    with pytest.raises(ValueError, match="goals"):
        ring.write_compact(0, pos[:A], act[:A], [1])
    with pytest.raises(ValueError, match="invalid action"):
        ring.write_compact(0, pos[:A], np.full(A, 5, np.uint8), [0])
    with pytest.raises(ValueError, match="out of bounds"):
        ring.write_compact(2, pos[:2 * A], act[:2 * A], [0, 0])
    with pytest.raises(ValueError, match="8 or 13"):
        CompactRingBuffer(12, 9, num_envs=3, agents_per_env=4)


def test_compact_ring_compacts_reference_producer_rows():
    """Producers that keep calling reserve_and_write(rows) fill the same slots."""
    E, A, S = 2, 3, 6
    _, arrays = make_compact(7, E, 16, A, S)
    stages = expand_records(*arrays, E, 13)
    ring = CompactRingBuffer(S * E * A, 13, num_envs=E, agents_per_env=A)
    for s in range(S):
        for e in range(E):
            ring.reserve_and_write(stages[s, e * A:(e + 1) * A].copy())
    for s in range(S):
        p, a, st, g = _decode_slot(ring, s)
        assert np.array_equal(p, arrays[0][s]) and np.array_equal(a, arrays[1][s])
        assert np.array_equal(st, arrays[2][s])
        for e in np.flatnonzero(st):
            k = int(np.cumsum(arrays[2].reshape(-1))[s * E + e] - 1)
            assert np.array_equal(g[e], arrays[3][k])
    bad = CompactRingBuffer(E * A, 13, num_envs=E, agents_per_env=A)
    row = stages[1, :A].copy()
    if row[0, 7] == 0:
        with pytest.raises(ValueError, match="start an episode first"):
            bad.reserve_and_write(row)
    first = stages[0, :A].copy()
    first[1, 8] = 1
    with pytest.raises(ValueError, match="previous actions"):
        bad.reserve_and_write(first)


@pytest.mark.parametrize("workers", [None, 2])
def test_ring_stage_source_streams_compact_records(tmp_path, workers):
    E, A, S = 4, 3, 7
    grids, arrays = make_compact(9, E, 16, A, S)
    stages = expand_records(*arrays, E, 13)
    save_compact_records(tmp_path / "c", backend="mapf_gpt", grids=grids, stages=stages, metadata={})
    ring = CompactRingBuffer(2 * E * A, 13, num_envs=E, agents_per_env=A)
    config = {"num_agents": A, "num_steps": S, "map_names": [f"m{e}" for e in range(E)]}
    src = RingStageSource(ring, "mapf_gpt", config, records=tmp_path / "c", timeout=30, workers=workers)
    try:
        assert len(src.processes) == (E if workers is None else 2)
        src.start()
        k = 0
        for s in range(S):
            deadline = 200
            while not ring.is_stage_ready(s):
                src.check()
                deadline -= 1
                assert deadline > 0, s
                import time
                time.sleep(0.05)
            p, a, st, g = _decode_slot(ring, s)
            assert np.array_equal(p, arrays[0][s]) and np.array_equal(a, arrays[1][s])
            assert np.array_equal(st, arrays[2][s])
            for e in np.flatnonzero(st):
                assert np.array_equal(g[e], arrays[3][k]), (s, e)
                k += 1
            ring.release_stage(s)
            ring.shared_compute_ptr.value = (s + 1) * ring.stage_rows
        with pytest.raises(RuntimeError, match="device"):
            src.next_rows()
    finally:
        src.close()
    # a compact archive cannot stream into a row ring
    with pytest.raises(ValueError, match="CompactRingBuffer"):
        RingStageSource(RingBuffer(E * A, 13, num_envs=E, agents_per_env=A), "mapf_gpt", config,
                        records=tmp_path / "c")
    m = json.loads((tmp_path / "c" / "manifest.json").read_text())
    assert m["goal_blocks"] == k
