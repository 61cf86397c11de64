"""HBM-resident expert-record ring: shared host ring -> pinned staging ->
hipMemcpyAsync on a side stream -> HBM ring -> the builders.

Same classes, constructor arguments, methods, attributes and error messages
as the reference's stage ring and its consumers, so producers and trainers
written against them run unchanged:

* ``RingBuffer``            expert_running.py:261-459
* ``DMAWorker``             expert_running.py:463-531
* ``GPUComputeHandler``     expert_running.py:537-551
* ``ExtremeMAPFPipeline``   expert_running.py:602-808 (MAGAT stages, 8 columns)
* ``MapfGPTOnlinePipeline`` mapf_gpt_online.py:97-184 (MAPF-GPT stages, 13 columns)
* ``validate_stage``        mapf_cuda/training/host_inputs.py:17-36
* ``save_records`` / ``load_records`` / ``RingStageSource``
                            mapf_cuda/training/frozen_stage_source.py:23-156

Producer side (unchanged protocol): each producer process reserves the next
stage slot for its env, copies its env block (A rows) into the shared host
ring and publishes it; a stage becomes visible only when every env has
published (fail-closed: a producer that dies after reserving leaves the
stage invisible; recovery is a whole-run restart).

Device side (this module's own design):

* ``cpu_buffer`` is plain shared memory.  The reference pins it and then
  shares it (``pin_memory().share_memory_()``, expert_running.py:295-297);
  sharing moves the storage into a fresh shared-memory mapping, and memory
  that already exists cannot be pinned after the fact here, so the DMA
  thread owns ``staging_slots`` pinned buffers of one stage each instead:
  a ready stage is copied shm -> pinned slot on the host, then the slot is
  copied into ``gpu_buffer`` (HBM, same capacity as the ring) with an
  asynchronous host-to-device copy on ``copy_stream``, and ``dma_event``
  (plus a per-slot event that guards the slot's reuse) is recorded.
* every stream keeps the default priority (the reference asks for a
  high-priority compute stream, expert_running.py:669; mixed stream
  priorities are avoided on this platform).
* the consumer orders its stream after ``dma_event``, copies the stage into
  ``stage_batch_buffer`` on the device, validates env/agent order and
  releases the stage so producers can reuse the slot.

Compact records (no reference counterpart; ``record_format="compact"`` of the
pipelines): ``CompactRingBuffer`` carries 5 bytes per agent-step (int16
position, uint8 action) plus per-env episode starts and the starting envs'
goals; ``CompactDMAWorker`` uploads a stage and expands it into the 8- or
13-column rows on the device in one native call (``jl_ring_upload_compact``),
so the consumer reads the same rows as from the row ring.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import multiprocessing as mp
import threading
import time
from pathlib import Path

import numpy as np
import torch

FEATURE_DIM = 8
MAPFGPT_FEATURE_DIM = 13
NUM_ACTIONS = 5
RESET_FLAG_COL = 7
_POLL_S = 0.0005
# the DMA thread's poll when the next stage is not complete yet: a stage of a
# large ring takes a few hundred microseconds end to end, so a 0.5 ms sleep
# would leave the device idle
_DMA_POLL_S = 0.00005


# ============================================================
# RingBuffer - shared host ring with the complete-stage protocol
# ============================================================
class RingBuffer:
    """Shared-memory ring of ``capacity`` rows x ``feature_dim`` int16.

    With ``num_envs`` and ``agents_per_env`` it is a stage ring: capacity is a
    multiple of one stage (num_envs * agents_per_env rows) and each producer
    writes one full env block per call (expert_running.py:261-459).
    """

    def __init__(
        self,
        capacity: int,
        feature_dim: int = FEATURE_DIM,
        *,
        num_envs: int | None = None,
        agents_per_env: int | None = None,
    ):
        self.capacity = capacity
        self.feature_dim = feature_dim
        self.num_envs = int(num_envs) if num_envs is not None else None
        self.agents_per_env = int(agents_per_env) if agents_per_env is not None else None
        self.stage_mode = self.num_envs is not None and self.agents_per_env is not None
        self.stage_rows = None
        self.num_stage_slots = None
        if self.stage_mode:
            if self.num_envs <= 0:
                raise ValueError(f"num_envs must be positive, got {self.num_envs}")
            if self.agents_per_env <= 0:
                raise ValueError(f"agents_per_env must be positive, got {self.agents_per_env}")
            self.stage_rows = self.num_envs * self.agents_per_env
            if capacity % self.stage_rows != 0:
                raise ValueError(
                    "stage-based ring capacity must be divisible by one frontier batch: "
                    f"capacity={capacity}, stage_rows={self.stage_rows}"
                )
            self.num_stage_slots = capacity // self.stage_rows
            if self.num_stage_slots <= 0:
                raise ValueError(
                    f"stage-based ring requires at least one stage slot, got capacity={capacity}"
                )
        # shared with forked producer processes; see the module docstring for pinning
        self.cpu_buffer = self._allocate_host_buffer()
        self.ready_flags = mp.Array("B", capacity)
        self._flags_view = None
        self.shared_reserve_ptr = mp.Value("Q", 0)
        self.shared_compute_ptr = mp.Value("Q", 0)
        self.reserve_lock = mp.Lock()
        if self.stage_mode:
            self.env_write_seq = mp.Array("Q", self.num_envs)
            self.stage_ready_counts = mp.Array("I", self.num_stage_slots)
            self.stage_seq_tags = mp.Array("q", [-1] * self.num_stage_slots)
        else:
            self.env_write_seq = None
            self.stage_ready_counts = None
            self.stage_seq_tags = None

    def _allocate_host_buffer(self) -> torch.Tensor:
        return torch.zeros((self.capacity, self.feature_dim), dtype=torch.int16).share_memory_()

    def _set_flags(self, start: int, end: int, value: int) -> None:
        """ready_flags[start:end] = value through a numpy view of the shared
        bytes (one memset instead of a Python list per call)."""
        if self._flags_view is None:
            self._flags_view = np.frombuffer(self.ready_flags.get_obj(), dtype=np.uint8)
        self._flags_view[start:end] = value

    def __getstate__(self):
        state = self.__dict__.copy()
        state["_flags_view"] = None
        return state

    def _stage_row_bounds(self, stage_seq: int, env_id: int | None = None) -> tuple[int, int]:
        if not self.stage_mode:
            raise RuntimeError("stage row bounds are only available in stage mode")
        stage_idx = int(stage_seq) % self.num_stage_slots
        row_start = stage_idx * self.stage_rows
        if env_id is not None:
            row_start += int(env_id) * self.agents_per_env
            return row_start, row_start + self.agents_per_env
        return row_start, row_start + self.stage_rows

    def _validate_stage_block(self, data: np.ndarray) -> tuple[int, torch.Tensor]:
        if data.ndim != 2 or data.shape[1] != self.feature_dim:
            raise ValueError(f"shape must be [N, {self.feature_dim}] in stage mode, got {data.shape}")
        if data.shape[0] != self.agents_per_env:
            raise ValueError(
                "stage-based ring expects one full env block per write: "
                f"expected {self.agents_per_env} rows, got {data.shape[0]}"
            )
        env_ids = data[:, 0]
        env_id = int(env_ids[0])
        if env_id < 0 or env_id >= self.num_envs:
            raise ValueError(
                f"env_id out of range for stage-based ring: env_id={env_id}, num_envs={self.num_envs}"
            )
        if not np.all(env_ids == env_id):
            raise ValueError("stage-based ring requires every written block to contain a single env_id")
        if not np.array_equal(data[:, 1], np.arange(self.agents_per_env, dtype=np.uint16)):
            raise ValueError("stage-based ring expects agent ids to be contiguous 0..agents_per_env-1")
        return env_id, torch.from_numpy(data.astype(np.int16, copy=False))

    def _reserve_stage_block(self, env_id: int) -> tuple[int, int, int]:
        """Reserve the env's next stage slot (installs the sequence tag only).

        The slot is free when the env is fewer than num_stage_slots stages
        ahead of the consumer and the slot's tag is empty, this stage's, or
        one the consumer has passed.  The stage stays invisible until every
        env has called ``_publish_stage_block``.
        """
        return self._reserve_stage_range(env_id, env_id + 1)

    def _reserve_stage_range(self, env_lo: int, env_hi: int) -> tuple[int, int, int]:
        """``_reserve_stage_block`` for the contiguous envs [env_lo, env_hi),
        written by one producer that keeps them at the same stage."""
        while True:
            with self.reserve_lock:
                seqs = self.env_write_seq[env_lo:env_hi]
                write_seq = int(seqs[0])
                if any(int(q) != write_seq for q in seqs):
                    raise ValueError("envs of one producer range are at different stages")
                consumed_seq = self.shared_compute_ptr.value // self.stage_rows
                if write_seq - consumed_seq < self.num_stage_slots:
                    stage_idx = write_seq % self.num_stage_slots
                    stage_tag = int(self.stage_seq_tags[stage_idx])
                    if stage_tag in (-1, write_seq) or stage_tag < consumed_seq:
                        if stage_tag != write_seq:
                            self.stage_seq_tags[stage_idx] = write_seq
                            self.stage_ready_counts[stage_idx] = 0
                        row_start = self._stage_row_bounds(write_seq, env_id=env_lo)[0]
                        return write_seq, row_start, row_start + (env_hi - env_lo) * self.agents_per_env
            time.sleep(_POLL_S)

    def _publish_stage_block(self, env_id: int, write_seq: int) -> None:
        """Publish one fully written env block into its stage."""
        self._publish_stage_range(env_id, env_id + 1, write_seq)

    def _publish_stage_range(self, env_lo: int, env_hi: int, write_seq: int) -> None:
        with self.reserve_lock:
            stage_idx = write_seq % self.num_stage_slots
            self.stage_ready_counts[stage_idx] += env_hi - env_lo
            self.env_write_seq[env_lo:env_hi] = [write_seq + 1] * (env_hi - env_lo)
            self.shared_reserve_ptr.value += (env_hi - env_lo) * self.agents_per_env

    def _stage_reserve_and_write(self, data: np.ndarray):
        env_id, block = self._validate_stage_block(data)
        write_seq, row_start, row_end = self._reserve_stage_block(env_id)
        self.cpu_buffer[row_start:row_end].copy_(block)
        self._set_flags(row_start, row_end, 1)
        self._publish_stage_block(env_id, write_seq)
        return (row_start, row_end)

    def reserve_and_write(self, data: np.ndarray):
        """Write rows (one env block in stage mode); blocks while the ring is full."""
        if self.stage_mode:
            return self._stage_reserve_and_write(data)
        n = data.shape[0]
        if n == 0:
            return (0, 0)
        if n > self.capacity:
            raise ValueError(f"cannot write chunk of size {n} into ring buffer capacity {self.capacity}")
        rows = torch.from_numpy(data.astype(np.int16, copy=False))
        while True:
            with self.reserve_lock:
                start_ptr = self.shared_reserve_ptr.value
                if start_ptr - self.shared_compute_ptr.value + n <= self.capacity:
                    self.shared_reserve_ptr.value += n
                    break
            time.sleep(_POLL_S)
        idx_start = start_ptr % self.capacity
        idx_end = (idx_start + n) % self.capacity
        if idx_start < idx_end or idx_end == 0:
            end = self.capacity if idx_end == 0 else idx_end
            self.cpu_buffer[idx_start:end].copy_(rows)
            self._set_flags(idx_start, end, 1)
            return (idx_start, end)
        first = self.capacity - idx_start
        self.cpu_buffer[idx_start:self.capacity].copy_(rows[:first])
        self.cpu_buffer[0:idx_end].copy_(rows[first:])
        self._set_flags(idx_start, self.capacity, 1)
        self._set_flags(0, idx_end, 1)
        return (idx_start, idx_end)

    def is_stage_ready(self, stage_seq: int) -> bool:
        if not self.stage_mode:
            return False
        stage_idx = int(stage_seq) % self.num_stage_slots
        with self.reserve_lock:
            return (
                int(self.stage_seq_tags[stage_idx]) == int(stage_seq)
                and int(self.stage_ready_counts[stage_idx]) >= self.num_envs
            )

    def release_stage(self, stage_seq: int) -> None:
        if not self.stage_mode:
            return
        row_start, row_end = self._stage_row_bounds(stage_seq)
        stage_idx = int(stage_seq) % self.num_stage_slots
        with self.reserve_lock:
            self.stage_ready_counts[stage_idx] = 0
            self.stage_seq_tags[stage_idx] = -1
        self._set_flags(row_start, row_end, 0)

    def scan_ready_range(self, start_ptr: int, max_scan: int) -> int:
        idx_start = start_ptr % self.capacity
        for i in range(max_scan):
            if self.ready_flags[idx_start + i] == 0:
                return i
        return max_scan

    def clear_flags(self, start: int, end: int) -> None:
        self._set_flags(start, end, 0)


# ============================================================
# DMAWorker - host ring -> pinned staging -> HBM ring
# ============================================================
class DMAWorker:
    """Moves ready rows of ``ring_buffer`` into ``gpu_buffer`` (expert_running.py:463-531)."""

    def __init__(self, ring_buffer: RingBuffer, gpu_buffer: torch.Tensor, batch_threshold=4096,
                 device="cuda:0", *, staging_slots: int = 2):
        self.ring_buffer = ring_buffer
        self.gpu_buffer = gpu_buffer
        self.batch_threshold = batch_threshold
        self.device = torch.device(device)
        self.copy_stream = torch.cuda.Stream(device=self.device)
        self.dma_event = torch.cuda.Event(enable_timing=False)
        self.dma_read_ptr = 0
        self._running = False
        rows = ring_buffer.stage_rows if ring_buffer.stage_mode else max(1, ring_buffer.capacity // 4)
        self.staging = [
            torch.empty((rows, ring_buffer.feature_dim), dtype=torch.int16).pin_memory()
            for _ in range(max(1, int(staging_slots)))
        ]
        self.staging_events = [None] * len(self.staging)
        self._slot = 0
        # set to a list to collect (bytes, upload events) per stage for measurement
        self.timing = None
        self.host_seconds = 0.0  # host time moving stages (staging copy + enqueue), waits excluded

    def _timing_event(self, stream):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(stream)
        return ev

    def _copy_rows(self, idx_start: int, idx_end: int) -> None:
        """cpu_buffer[idx_start:idx_end] -> gpu_buffer[idx_start:idx_end] through a pinned slot."""
        slot = self._slot
        self._slot = (slot + 1) % len(self.staging)
        pending = self.staging_events[slot]
        if pending is not None:
            pending.synchronize()  # the slot's previous upload has left host memory
        t_host = time.perf_counter()
        n = idx_end - idx_start
        staged = self.staging[slot][:n]
        staged.copy_(self.ring_buffer.cpu_buffer[idx_start:idx_end])
        with torch.cuda.stream(self.copy_stream):
            t0 = self._timing_event(self.copy_stream) if self.timing is not None else None
            self.gpu_buffer[idx_start:idx_end].copy_(staged, non_blocking=True)
            if t0 is not None:
                self.timing.append((staged.numel() * staged.element_size(), t0,
                                    self._timing_event(self.copy_stream), None))
            done = torch.cuda.Event(enable_timing=False)
            done.record(self.copy_stream)
            self.dma_event.record(self.copy_stream)
        self.staging_events[slot] = done
        self.host_seconds += time.perf_counter() - t_host

    def run_once(self):
        ring = self.ring_buffer
        if ring.stage_mode:
            stage_seq = self.dma_read_ptr // ring.stage_rows
            if not ring.is_stage_ready(stage_seq):
                return None
            idx_start, idx_end = ring._stage_row_bounds(stage_seq)
            self._copy_rows(idx_start, idx_end)
            self.dma_read_ptr += ring.stage_rows
            return (idx_start, idx_end)
        available = ring.shared_reserve_ptr.value - self.dma_read_ptr
        if available <= 0:
            return None
        idx_start = self.dma_read_ptr % ring.capacity
        max_scan = min(available, ring.capacity - idx_start, ring.capacity // 4,
                       self.staging[0].shape[0])
        ready = ring.scan_ready_range(self.dma_read_ptr, max_scan)
        if ready <= 0:
            return None
        idx_end = idx_start + ready
        self._copy_rows(idx_start, idx_end)
        ring.clear_flags(idx_start, idx_end)
        self.dma_read_ptr += ready
        return (idx_start, idx_end)

    def release_completed_stage(self, stage_seq: int) -> None:
        if not self.ring_buffer.stage_mode:
            return
        self.ring_buffer.release_stage(stage_seq)
        self.ring_buffer.shared_compute_ptr.value = (int(stage_seq) + 1) * self.ring_buffer.stage_rows

    def start(self):
        self._running = True
        t = threading.Thread(target=self._loop, daemon=True)
        t.start()
        return t

    def stop(self):
        self._running = False

    def _loop(self):
        while self._running:
            if self.run_once() is None:
                time.sleep(_DMA_POLL_S)


# ============================================================
# Compact stage ring - 5 bytes per agent and step over the host link
# ============================================================
def _align(n: int, a: int) -> int:
    return (n + a - 1) // a * a


class CompactRingBuffer(RingBuffer):
    """Stage ring whose slots hold compact records (records.py) instead of rows.

    Same stage protocol, sequence tags, counters and pointers (counted in rows)
    as ``RingBuffer``; a slot of N = num_envs * agents_per_env agents is::

        [0, 4N)                 positions   uint16 [N, 2]
        [4N, 5N)                actions     uint8  [N]
        [5N, 5N + E)            episode start flags, one byte per env
        [goals, goals + 4N)     goals       uint16 [N, 2], written for starting envs only

    ``cpu_buffer`` is uint8 [num_stage_slots, slot_bytes].  Producers either
    call ``write_compact`` with compact blocks or keep calling
    ``reserve_and_write`` with full env blocks (the reference producer API):
    those are compacted here, and rows that the compact form cannot carry
    (records.py) raise ValueError in the producer.
    """

    def __init__(self, capacity: int, feature_dim: int = FEATURE_DIM, *, num_envs: int, agents_per_env: int):
        if feature_dim not in (FEATURE_DIM, MAPFGPT_FEATURE_DIM):
            raise ValueError(f"feature_dim must be {FEATURE_DIM} or {MAPFGPT_FEATURE_DIM}, got {feature_dim}")
        n = int(num_envs) * int(agents_per_env)
        self.off_actions = 4 * n
        self.off_starts = 5 * n
        self.head_bytes = 5 * n + int(num_envs)
        self.off_goals = _align(self.head_bytes, 16)
        self.slot_bytes = _align(self.off_goals + 4 * n, 64)
        super().__init__(capacity, feature_dim, num_envs=num_envs, agents_per_env=agents_per_env)
        self._tracked = {}  # producer-side: env -> (goals, history) of its running episode

    def _allocate_host_buffer(self) -> torch.Tensor:
        if not self.stage_mode:
            raise ValueError("a compact ring needs num_envs and agents_per_env")
        return torch.zeros((self.num_stage_slots, self.slot_bytes), dtype=torch.uint8).share_memory_()

    def slot_view(self, stage_seq: int) -> np.ndarray:
        """uint8 view of the host slot of a stage."""
        return self.cpu_buffer[int(stage_seq) % self.num_stage_slots].numpy()

    def write_compact(self, env_lo: int, positions, actions, episode_start, goals=None):
        """Write the compact blocks of the contiguous envs [env_lo, env_lo + n)
        (n = len(episode_start)) into their next stage with one reservation.
        ``positions`` [n*A, 2] and ``goals`` [n*A, 2] are 16-bit, ``actions``
        [n*A] 0..4; goals are required when any env starts an episode."""
        A = self.agents_per_env
        starts = np.asarray(episode_start, dtype=np.uint8).reshape(-1)
        n_env = starts.shape[0]
        env_lo = int(env_lo)
        if n_env <= 0 or env_lo < 0 or env_lo + n_env > self.num_envs:
            raise ValueError(f"env range out of bounds: [{env_lo}, {env_lo + n_env}) of {self.num_envs}")
        pos = np.asarray(positions)
        act = np.asarray(actions)
        if pos.shape != (n_env * A, 2) or act.shape != (n_env * A,):
            raise ValueError(f"compact block must hold {n_env * A} positions [.,2] and actions")
        if np.any(act > 4) or np.any(starts > 1):
            raise ValueError("invalid action or refresh flag")
        if starts.any():
            if goals is None or np.asarray(goals).shape != (n_env * A, 2):
                raise ValueError("goals [n*A, 2] are required for envs that start an episode")
        write_seq, row_start, row_end = self._reserve_stage_range(env_lo, env_lo + n_env)
        slot = self.slot_view(write_seq)
        a0, a1 = env_lo * A, (env_lo + n_env) * A
        slot[4 * a0:4 * a1].view(np.uint16)[:] = pos.astype(np.uint16, copy=False).reshape(-1)
        slot[self.off_actions + a0:self.off_actions + a1] = act
        slot[self.off_starts + env_lo:self.off_starts + env_lo + n_env] = starts
        if starts.any():
            g = np.asarray(goals).astype(np.uint16, copy=False).reshape(n_env, A * 2)
            dst = slot[self.off_goals + 4 * a0:self.off_goals + 4 * a1].view(np.uint16).reshape(n_env, A * 2)
            dst[starts == 1] = g[starts == 1]
        self._set_flags(row_start, row_end, 1)
        self._publish_stage_range(env_lo, env_lo + n_env, write_seq)
        return (row_start, row_end)

    def _stage_reserve_and_write(self, data: np.ndarray):
        """A full env block (reference producer API), compacted."""
        if data.ndim != 2 or data.shape[1] != self.feature_dim:
            raise ValueError(f"shape must be [N, {self.feature_dim}] in stage mode, got {data.shape}")
        env_id, _ = self._validate_stage_block(data)
        rows = data.astype(np.int64)
        refresh = rows[:, RESET_FLAG_COL]
        if np.any(refresh > 1) or np.any(rows[:, 6] > 4):
            raise ValueError("invalid action or refresh flag")
        start = int(refresh[0])
        if np.any(refresh != start):
            raise ValueError("compact records need one refresh flag per env and stage")
        goals = rows[:, 4:6]
        tracked = self._tracked.get(env_id)
        if start:
            history = np.full((self.agents_per_env, 5), 5, np.int64)
        else:
            if tracked is None:
                raise ValueError("compact records need every env to start an episode first")
            if not np.array_equal(goals, tracked[0]):
                raise ValueError("compact records need goals that change only at an episode start")
            history = tracked[1]
        if self.feature_dim == MAPFGPT_FEATURE_DIM and not np.array_equal(rows[:, 8:13], history):
            raise ValueError("history columns are not the previous actions of the episode")
        history = np.concatenate([history[:, 1:], rows[:, 6:7]], axis=1)
        out = self.write_compact(env_id, rows[:, 2:4], rows[:, 6], [start], goals if start else None)
        self._tracked[env_id] = (goals, history)
        return out


class CompactDMAWorker(DMAWorker):
    """Moves ready compact stages to the device and expands them there into
    ``gpu_buffer`` rows (the same rows a row ring would deliver).

    Per stage one native call (``jl_ring_upload_compact``, run without the
    interpreter lock) copies the slot's head (positions, actions, start
    flags: 5N + E bytes) and the goal range of the envs that start an
    episode from the shared host ring into a pinned staging buffer, uploads
    them on ``copy_stream``, waits on the device for the consumer's copy out
    of the ring slot's rows, expands the stage into ``gpu_buffer`` (advancing
    the running goals and histories) and records ``dma_event``."""

    def __init__(self, ring_buffer: CompactRingBuffer, gpu_buffer: torch.Tensor, batch_threshold=4096,
                 device="cuda:0", *, staging_slots: int = 2):
        from ._abi import StageUploadDesc, load_library
        from .records import RecordExpander

        if not isinstance(ring_buffer, CompactRingBuffer):
            raise TypeError("CompactDMAWorker needs a CompactRingBuffer")
        self.ring_buffer = ring_buffer
        self.gpu_buffer = gpu_buffer
        self.batch_threshold = batch_threshold
        self.device = torch.device(device)
        self._lib = load_library()
        self.copy_stream = torch.cuda.Stream(device=self.device)
        k = max(1, int(staging_slots))
        L = ring_buffer.slot_bytes
        self.staging = [torch.empty(L, dtype=torch.uint8).pin_memory() for _ in range(k)]
        self.device_slots = torch.empty((k, L), dtype=torch.uint8, device=self.device)
        self.dma_read_ptr = 0
        self._running = False
        self._slot = 0
        self.expander = RecordExpander(ring_buffer.num_envs, ring_buffer.agents_per_env,
                                       ring_buffer.feature_dim, self.device)
        # events the native step records and waits on: created here (a first
        # record), re-recorded by the library
        self.dma_event = torch.cuda.Event(enable_timing=False)
        self.staging_events = [torch.cuda.Event(enable_timing=False) for _ in range(k)]
        # per ring slot: recorded after the consumer's copy out of the slot's rows
        self._consumed = [torch.cuda.Event(enable_timing=False) for _ in range(ring_buffer.num_stage_slots)]
        self._consumed_used = [False] * ring_buffer.num_stage_slots
        for ev in [self.dma_event, *self.staging_events, *self._consumed]:
            ev.record(self.copy_stream)
        self.bytes_uploaded = 0
        self.host_seconds = 0.0  # host time of the native step (staging copy + enqueue), waits included
        # set to a list to collect (bytes, start event, end event) of upload + expansion per stage
        self.timing = None
        u = StageUploadDesc()
        u.slot_bytes = L
        u.records = self.expander._desc  # sizes, running goals and histories (a copy of the struct)
        u.done = self.dma_event.cuda_event
        self._upload = u
        self._host_ptrs = [ring_buffer.cpu_buffer[j].data_ptr() for j in range(ring_buffer.num_stage_slots)]
        self._rows_ptrs = [gpu_buffer[ring_buffer._stage_row_bounds(j)[0]].data_ptr()
                           for j in range(ring_buffer.num_stage_slots)]

    def mark_slot_consumed(self, stage_seq: int, stream) -> None:
        """Record on the consumer's stream that the stage's rows have been
        copied out of ``gpu_buffer``: the slot's next expansion waits for it."""
        j = int(stage_seq) % len(self._consumed)
        self._consumed[j].record(stream)
        self._consumed_used[j] = True

    def _copy_stage(self, stage_seq: int) -> tuple[int, int]:
        from ._abi import check

        t_host = time.perf_counter()
        ring = self.ring_buffer
        slot = self._slot
        self._slot = (slot + 1) % len(self.staging)
        j = int(stage_seq) % ring.num_stage_slots
        u = self._upload
        u.host_slot = self._host_ptrs[j]
        u.staging = self.staging[slot].data_ptr()
        u.device_slot = self.device_slots[slot].data_ptr()
        u.staging_free = self.staging_events[slot].cuda_event
        u.rows_free = self._consumed[j].cuda_event if self._consumed_used[j] else None
        u.records.rows = self._rows_ptrs[j]
        t0 = self._timing_event(self.copy_stream) if self.timing is not None else None
        check(self._lib.jl_ring_upload_compact(ctypes.byref(u), self.copy_stream.cuda_stream),
              "compact stage upload")
        if t0 is not None:
            self.timing.append((u.bytes_uploaded, t0, self._timing_event(self.copy_stream)))
        self.bytes_uploaded += u.bytes_uploaded
        self.host_seconds += time.perf_counter() - t_host
        return ring._stage_row_bounds(stage_seq)

    def run_once(self):
        ring = self.ring_buffer
        stage_seq = self.dma_read_ptr // ring.stage_rows
        if not ring.is_stage_ready(stage_seq):
            return None
        bounds = self._copy_stage(stage_seq)
        self.dma_read_ptr += ring.stage_rows
        return bounds


# ============================================================
# GPUComputeHandler
# ============================================================
class GPUComputeHandler:
    """MAGAT stage refresh (expert_running.py:537-551)."""

    def __init__(self, simulator):
        self.simulator = simulator

    def process_batch(self, full_batch: torch.Tensor, agents_to_update: torch.Tensor):
        if agents_to_update.shape[0] > 0:
            self.simulator.update_derived_state(agents_to_update, agents_to_update.shape[0])
        self.simulator.refresh_compact_state_from_raw_batch(full_batch)

    def filter_reset_agents(self, full_batch: torch.Tensor) -> torch.Tensor:
        return full_batch[full_batch[:, RESET_FLAG_COL] != 0]


# ============================================================
# ExtremeMAPFPipeline - MAGAT stage consumer
# ============================================================
class ExtremeMAPFPipeline:
    """Ring + DMA + stage consumer for a MAGAT simulator (expert_running.py:602-808)."""

    def __init__(self, simulator, capacity=16384 * 128, batch_threshold=16384,
                 feature_dim=FEATURE_DIM, device="cuda:0", *, record_format: str = "rows"):
        if record_format not in ("rows", "compact"):
            raise ValueError(f"record_format must be 'rows' or 'compact', got {record_format!r}")
        self.record_format = record_format
        self.device = torch.device(device)
        self.capacity = capacity
        self.batch_threshold = batch_threshold
        self.feature_dim = feature_dim
        self.cuda_simulator = simulator
        self.ring_buffer = None
        self.gpu_buffer = None
        self.gpu_handler = None
        self.dma_worker = None
        self.dma_read_ptr = 0
        self.compute_ptr = 0
        self.dma_event = None
        self.compute_stream = None
        self.graph_rows = None
        self.stage_batch_buffer = None
        self.expected_agent_ids_cache = {}
        self.stage_mode = False
        self.agents_per_env = None
        self.num_envs = None

    def _infer_stage_layout(self) -> tuple[int | None, int | None]:
        pyg_ptr = getattr(self.cuda_simulator, "pyg_ptr", None)
        if pyg_ptr is None or pyg_ptr.shape[0] <= 1:
            return None, None
        agents_per_env = int((pyg_ptr[1] - pyg_ptr[0]).item())
        num_envs = int(pyg_ptr.shape[0] - 1)
        if agents_per_env <= 0 or num_envs <= 0:
            return None, None
        return agents_per_env, num_envs

    def _make_ring(self, feature_dim: int) -> None:
        compact = self.record_format == "compact"
        ring_cls = CompactRingBuffer if compact else RingBuffer
        self.ring_buffer = ring_cls(self.capacity, feature_dim, num_envs=self.num_envs,
                                    agents_per_env=self.agents_per_env)
        self.gpu_buffer = torch.zeros((self.capacity, feature_dim), dtype=torch.int16, device=self.device)
        stage_rows = self.ring_buffer.stage_rows if self.ring_buffer.stage_mode else self.batch_threshold
        self.stage_batch_buffer = torch.empty((stage_rows, feature_dim), dtype=torch.int16, device=self.device)
        dma_cls = CompactDMAWorker if compact else DMAWorker
        self.dma_worker = dma_cls(self.ring_buffer, self.gpu_buffer, self.batch_threshold, str(self.device))
        self.dma_event = self.dma_worker.dma_event
        self.compute_stream = torch.cuda.Stream(device=self.device)

    def initialize(self):
        self.agents_per_env, self.num_envs = self._infer_stage_layout()
        self.stage_mode = self.agents_per_env is not None and self.num_envs is not None
        self._make_ring(self.feature_dim)
        self.gpu_handler = GPUComputeHandler(self.cuda_simulator)
        self.graph_rows = int(self.cuda_simulator.pyg_batch.shape[0])
        return self

    def reserve_and_write(self, transitions_numpy):
        if self.ring_buffer is None:
            raise RuntimeError("Pipeline not initialized. Call initialize() first.")
        return self.ring_buffer.reserve_and_write(transitions_numpy)

    def dma_worker_loop(self):
        if self.dma_worker is None:
            raise RuntimeError("Pipeline not initialized. Call initialize() first.")
        self.dma_worker.start()

    def _expected_agent_ids(self, agents_per_env: int, device: torch.device) -> torch.Tensor:
        key = (agents_per_env, device.type, device.index)
        expected = self.expected_agent_ids_cache.get(key)
        if expected is None:
            expected = torch.arange(agents_per_env, dtype=torch.int16, device=device)
            self.expected_agent_ids_cache[key] = expected
        return expected

    def _validate_env_aligned_batch(self, raw_batch: torch.Tensor, agents_per_env: int, num_envs: int) -> None:
        if raw_batch.shape[0] != agents_per_env * num_envs:
            raise ValueError(
                "env-aligned batch size mismatch: "
                f"expected {agents_per_env * num_envs}, got {raw_batch.shape[0]}"
            )
        blocks = raw_batch.view(num_envs, agents_per_env, raw_batch.shape[1])
        env_ids = blocks[:, :, 0].to(torch.int64)
        expected_env = torch.arange(num_envs, dtype=torch.int64, device=raw_batch.device)
        if not torch.all(env_ids == expected_env.view(num_envs, 1)):
            raise ValueError("stage-based frontier batch must be strict env-major with one block per env")
        expected_agents = self._expected_agent_ids(agents_per_env, raw_batch.device)
        if not torch.all(blocks[:, :, 1] == expected_agents.unsqueeze(0)):
            raise ValueError(
                "stage-based frontier batch expects agent ids to be contiguous 0..agents_per_env-1"
            )

    def has_env_aligned_batch(self, num_envs: int) -> bool:
        if self.ring_buffer is None or not self.ring_buffer.stage_mode:
            return False
        return self.ring_buffer.is_stage_ready(self.compute_ptr // self.ring_buffer.stage_rows)

    def extract_env_aligned_batch(self, chunk_size: int, agents_per_env: int, num_envs: int) -> torch.Tensor:
        """Device copy of the next complete stage (or None), then release its slot."""
        if self.ring_buffer is None or not self.ring_buffer.stage_mode:
            return None
        stage_seq = self.compute_ptr // self.ring_buffer.stage_rows
        if not self.ring_buffer.is_stage_ready(stage_seq):
            return None
        chunk_size = agents_per_env * num_envs
        dma_available = 0 if self.dma_worker is None else int(self.dma_worker.dma_read_ptr - self.compute_ptr)
        if dma_available < chunk_size:
            return None
        row_start, row_end = self.ring_buffer._stage_row_bounds(stage_seq)
        if self.stage_batch_buffer is None or self.stage_batch_buffer.shape[0] < chunk_size:
            self.stage_batch_buffer = torch.empty((chunk_size, self.gpu_buffer.shape[1]),
                                                  dtype=self.gpu_buffer.dtype, device=self.gpu_buffer.device)
        raw_batch = self.stage_batch_buffer[:chunk_size]
        # ordered after the stage's upload by the caller's wait on dma_event
        torch.cuda.current_stream(self.gpu_buffer.device).wait_event(self.dma_event)
        raw_batch.copy_(self.gpu_buffer[row_start:row_end], non_blocking=False)
        if isinstance(self.dma_worker, CompactDMAWorker):
            # env and agent ids were written by the device expansion from the
            # row index, so there is nothing to validate; the slot's next
            # expansion is ordered after this copy on the device instead of
            # by a host synchronisation
            self.dma_worker.mark_slot_consumed(stage_seq, torch.cuda.current_stream(self.gpu_buffer.device))
        else:
            self._validate_env_aligned_batch(raw_batch, agents_per_env, num_envs)
        self.compute_ptr += chunk_size
        self.dma_worker.release_completed_stage(stage_seq)
        return raw_batch

    def _layout(self) -> tuple[int, int]:
        ptr = self.cuda_simulator.pyg_ptr
        agents_per_env = int((ptr[1] - ptr[0]).item()) if ptr.shape[0] > 1 else 0
        return agents_per_env, int(ptr.shape[0] - 1)

    def train_step(self, model=None, optimizer=None, runtime=None):
        if self.dma_worker is None:
            return None
        agents_per_env, num_envs = self._layout()
        raw_batch = self.extract_env_aligned_batch(agents_per_env * num_envs, agents_per_env=agents_per_env,
                                                   num_envs=num_envs)
        if raw_batch is None:
            return None
        agents_to_update = self.gpu_handler.filter_reset_agents(raw_batch)
        self.gpu_handler.process_batch(raw_batch, agents_to_update)
        if runtime is not None:
            return runtime.train_step(self.cuda_simulator, raw_batch)
        if model is not None:
            loss = model(self.cuda_simulator.pyg_x)
            if optimizer is not None:
                optimizer.zero_grad(set_to_none=True)
                loss.backward()
                optimizer.step()
            return loss
        return self.cuda_simulator.pyg_x

    def get_stats(self):
        ring = self.ring_buffer
        stats = {
            "capacity": self.capacity,
            "reserve_ptr": ring.shared_reserve_ptr.value if ring else 0,
            "dma_read_ptr": self.dma_worker.dma_read_ptr if self.dma_worker is not None else self.dma_read_ptr,
            "compute_ptr": self.compute_ptr,
        }
        if ring is not None and ring.stage_mode:
            stats.update({
                "num_stage_slots": ring.num_stage_slots,
                "stage_rows": ring.stage_rows,
                "stage_ready_counts": list(ring.stage_ready_counts),
                "stage_seq_tags": list(ring.stage_seq_tags),
                "env_write_stage": list(ring.env_write_seq),
            })
        return stats

    def shutdown(self):
        if self.dma_worker is not None:
            self.dma_worker.stop()

    def __del__(self):
        self.shutdown()


# ============================================================
# MapfGPTOnlinePipeline - MAPF-GPT stage consumer
# ============================================================
class MapfGPTOnlinePipeline(ExtremeMAPFPipeline):
    """13-column stages into a MapfGPTObservationBuilder (mapf_gpt_online.py:97-184)."""

    def __init__(self, builder, runtime, *, capacity: int, batch_threshold: int, device: str = "cuda:0",
                 record_format: str = "rows"):
        super().__init__(builder, capacity=capacity, batch_threshold=batch_threshold,
                         feature_dim=MAPFGPT_FEATURE_DIM, device=device, record_format=record_format)
        self.runtime = runtime

    def initialize(self):
        self.agents_per_env, self.num_envs = self._infer_stage_layout()
        if self.agents_per_env is None or self.num_envs is None:
            raise ValueError("MAPF-GPT builder must expose a non-empty pyg_ptr stage layout")
        self.stage_mode = True
        stage_rows = self.agents_per_env * self.num_envs
        if self.batch_threshold != stage_rows:
            raise ValueError(
                "MAPF-GPT online pipeline requires one complete frontier per batch: "
                f"expected {stage_rows}, got {self.batch_threshold}"
            )
        self._make_ring(MAPFGPT_FEATURE_DIM)
        self.gpu_handler = None
        self.graph_rows = int(self.cuda_simulator.tokens.shape[0])
        return self

    def consume_once(self, *, capture_stage_hash: bool = False):
        if self.dma_worker is None:
            raise RuntimeError("Pipeline not initialized. Call initialize() first.")
        if not self.has_env_aligned_batch(self.num_envs):
            return None
        stage_rows = self.agents_per_env * self.num_envs
        if self.dma_worker.dma_read_ptr - self.compute_ptr < stage_rows:
            return None
        with torch.cuda.stream(self.compute_stream):
            raw_stage = self.extract_env_aligned_batch(stage_rows, agents_per_env=self.agents_per_env,
                                                       num_envs=self.num_envs)
            if raw_stage is None:
                return None
            stage_sha256 = None
            if capture_stage_hash:
                stage_sha256 = hashlib.sha256(raw_stage.detach().cpu().contiguous().numpy().tobytes()).hexdigest()
            metrics = self.runtime.train_step(self.cuda_simulator, raw_stage)
            if stage_sha256 is not None:
                metrics["stage_sha256"] = stage_sha256
            return metrics


# ============================================================
# Frozen expert records
# ============================================================
def validate_stage(rows, grids, agents, features):
    """Complete env-major uint16 stage of valid records (host_inputs.py:17-36)."""
    rows = np.asarray(rows)
    if rows.dtype != np.uint16 or rows.shape != (len(grids) * agents, features):
        raise ValueError("stage must contain complete uint16 environment-major records")
    blocks = rows.reshape(len(grids), agents, features)
    if not np.array_equal(blocks[:, :, 0], np.broadcast_to(np.arange(len(grids))[:, None], blocks.shape[:2])):
        raise ValueError("stage environment order mismatch")
    if not np.array_equal(blocks[:, :, 1], np.broadcast_to(np.arange(agents), blocks.shape[:2])):
        raise ValueError("stage agent order mismatch")
    if np.any(rows[:, 6] > 4) or np.any(rows[:, 7] > 1):
        raise ValueError("invalid action or refresh flag")
    for grid, block in zip(grids, blocks):
        for coords in (block[:, 2:4], block[:, 4:6]):
            if np.any(coords[:, 0] >= grid.shape[0]) or np.any(coords[:, 1] >= grid.shape[1]):
                raise ValueError("coordinates outside map")
            if np.any(grid[coords[:, 0], coords[:, 1]]):
                raise ValueError("coordinates on obstacles")
            if len(np.unique(coords, axis=0)) != agents:
                raise ValueError("duplicate joint positions or goals")
    return blocks


def sha256_file(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1024 * 1024), b""):
            h.update(chunk)
    return h.hexdigest()


def save_records(output, *, backend, grids, stages, metadata):
    """Write grids.npy / stages.npy / manifest.json with sha256 (frozen_stage_source.py:23-42)."""
    output = Path(output)
    output.mkdir(parents=True, exist_ok=False)
    stages = np.asarray(stages)
    if not np.issubdtype(stages.dtype, np.integer) or np.any(stages < 0) or np.any(stages > 65535):
        raise ValueError("records must contain uint16-representable integers")
    stages = stages.astype(np.uint16)
    features = FEATURE_DIM if backend == "magat" else MAPFGPT_FEATURE_DIM
    if stages.ndim != 3 or not len(stages) or stages.shape[1] % len(grids):
        raise ValueError("invalid stage archive")
    agents = stages.shape[1] // len(grids)
    for rows in stages:
        validate_stage(rows, grids, agents, features)
    np.save(output / "grids.npy", np.asarray(grids, dtype=np.uint8), allow_pickle=False)
    np.save(output / "stages.npy", stages, allow_pickle=False)
    manifest = dict(schema_version=1, backend=backend, agents=agents, stages=len(stages), features=features,
                    metadata=metadata,
                    hashes={name: sha256_file(output / name) for name in ("grids.npy", "stages.npy")})
    (output / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest


def load_records(root):
    """Verify hashes and shapes; stages are memory-mapped (frozen_stage_source.py:45-59)."""
    root = Path(root)
    m = json.loads((root / "manifest.json").read_text())
    if m.get("schema_version") != 1 or set(m.get("hashes", {})) != {"grids.npy", "stages.npy"}:
        raise ValueError("unsupported or incomplete record manifest")
    for name, expected in m["hashes"].items():
        if sha256_file(root / name) != expected:
            raise ValueError(f"record hash mismatch: {name}")
    grids = np.load(root / "grids.npy", allow_pickle=False)
    stages = np.load(root / "stages.npy", mmap_mode="r", allow_pickle=False)
    if stages.shape != (m["stages"], len(grids) * m["agents"], m["features"]):
        raise ValueError("record shape differs from manifest")
    for rows in stages:
        validate_stage(rows, grids, m["agents"], m["features"])
    return m, grids, stages


class _WorkerGate:
    def __init__(self, ready, go, stop):
        self.ready, self.go, self.stop = ready, go, stop

    def mark_ready(self):
        self.ready.set()
        self.go.wait()

    def mark_complete_and_wait(self):
        self.stop.wait()


def _produce(envs, ring, backend, config, records, gate):
    """One producer: stream the blocks of envs [lo, hi) of every frozen stage
    into the ring, stage by stage."""
    if records is None:
        raise NotImplementedError("live expert producers (LaCAM + POGEMA) are not part of this build")
    lo, hi = envs
    a = config["num_agents"]
    n = config["num_steps"]
    if isinstance(ring, CompactRingBuffer) and _is_compact(records):
        from .records import CompactRecords

        arrays = {name: np.load(Path(records) / f"{name}.npy", mmap_mode="r", allow_pickle=False)
                  for name in ("positions", "actions", "episode_starts", "goals")}
        rec = CompactRecords(**arrays)
        goals = np.zeros(((hi - lo) * a, 2), np.uint16)
        gate.mark_ready()
        for s in range(min(n, rec.num_stages)):
            starts = np.asarray(rec.episode_starts[s, lo:hi])
            for k in np.flatnonzero(starts):
                goals[k * a:(k + 1) * a] = rec.env_goals(s, lo + int(k))
            ring.write_compact(lo, rec.positions[s, lo * a:hi * a], rec.actions[s, lo * a:hi * a], starts,
                               goals if starts.any() else None)
        gate.mark_complete_and_wait()
        return
    stages = np.load(Path(records) / "stages.npy", mmap_mode="r", allow_pickle=False)
    gate.mark_ready()
    for stage in stages[:n]:
        for e in range(lo, hi):
            ring.reserve_and_write(np.array(stage[e * a:(e + 1) * a], copy=True))
    gate.mark_complete_and_wait()


def _is_compact(records) -> bool:
    from .records import is_compact_archive

    return is_compact_archive(records)


class RingStageSource:
    """Producer processes streaming frozen records (frozen_stage_source.py:105-156).

    As in the reference, by default one process per env; ``workers`` (an
    addition) runs that many processes instead, each owning a contiguous env
    range, for archives with more envs than host cores.  Compact archives
    (records.py) stream into a ``CompactRingBuffer``: one compact write per
    worker and stage."""

    def __init__(self, ring, backend, config, *, records=None, timeout=120, workers=None):
        self.ring, self.timeout, self.seq = ring, timeout, 0
        self.count = config["num_steps"]
        n_env = len(config["map_names"])
        if records is not None and _is_compact(records) and not isinstance(ring, CompactRingBuffer):
            raise ValueError("compact records stream through a CompactRingBuffer (record_format='compact')")
        workers = n_env if workers is None else max(1, min(int(workers), n_env))
        bounds = [(w * n_env // workers, (w + 1) * n_env // workers) for w in range(workers)]
        ctx = mp.get_context("fork")
        self.go, self.stop = ctx.Event(), ctx.Event()
        self.ready = [ctx.Event() for _ in bounds]
        self.processes = [
            ctx.Process(target=_produce, args=(envs, ring, backend, config, records,
                                               _WorkerGate(ready, self.go, self.stop)), daemon=True)
            for envs, ready in zip(bounds, self.ready)
        ]
        for p in self.processes:
            p.start()
        try:
            deadline = time.monotonic() + timeout
            while not all(e.is_set() for e in self.ready):
                self.check()
                if time.monotonic() > deadline:
                    raise TimeoutError("expert initialization timeout")
                time.sleep(0.01)
        except BaseException:
            self.close()
            raise

    def check(self):
        if any(p.exitcode is not None for p in self.processes):
            raise RuntimeError(f"expert process exited: {[p.exitcode for p in self.processes]}")

    def start(self):
        self.go.set()

    def next_rows(self):
        """Host copy of the next complete stage (the CPU consumer of the same ring)."""
        if isinstance(self.ring, CompactRingBuffer):
            raise RuntimeError("compact stages are expanded on the device: consume them through the pipeline")
        if self.seq >= self.count:
            raise StopIteration
        deadline = time.monotonic() + self.timeout
        while not self.ring.is_stage_ready(self.seq):
            self.check()
            if time.monotonic() > deadline:
                raise TimeoutError("expert failed to publish a complete stage")
            time.sleep(_POLL_S)
        lo, hi = self.ring._stage_row_bounds(self.seq)
        result = self.ring.cpu_buffer[lo:hi].numpy().astype(np.uint16, copy=True)
        self.ring.release_stage(self.seq)
        self.seq += 1
        self.ring.shared_compute_ptr.value = self.seq * self.ring.stage_rows
        return result

    def close(self):
        self.stop.set()
        self.go.set()
        for p in self.processes:
            if p.is_alive():
                p.terminate()
            p.join(timeout=5)
