"""Expert-record ring: producers -> shared host stage ring -> pinned staging
-> HBM ring -> the builders.

The names callers use are the reference's, so producers and trainers written
against its ring run unchanged. That covers classes, constructor arguments,
the attributes they read, error messages, the stage-protocol fields and the
archive format:

* ``RingBuffer``             expert_running.py:261-459
* ``DMAWorker``              expert_running.py:463-531
* ``GPUComputeHandler``      expert_running.py:537-551
* ``ExtremeMAPFPipeline``    expert_running.py:602-808 (MAGAT stages, 8 columns)
* ``MapfGPTOnlinePipeline``  mapf_gpt_online.py:97-184 (MAPF-GPT stages, 13 columns)
* ``validate_stage``         mapf_cuda/training/host_inputs.py:17-36
* ``save_records`` / ``load_records`` / ``RingStageSource``
                             mapf_cuda/training/frozen_stage_source.py:23-156

The machinery underneath is this module's own.

Host ring without a lock on the stage path.  Every counter of a ring lives
in one shared int64 control block: the two row pointers, one word per env
(the number of stages that env has published: ``env_write_seq``) and one tag
per stage slot (the stage it holds, -1 when free: ``stage_seq_tags``).
Each env has exactly one producer, and each word has one writer:

* a producer writes its env block, then stores its env word;
* the consumer moves the compute pointer;
* a slot's tag is written only by the producers of the one stage that can
  hold the slot (all with the same value) and by the release of the stage
  before it, which the compute pointer orders.

A stage is complete when every env word has passed it (a vectorised
minimum); ``stage_ready_counts`` is derived from the same words.  The host
is x86-64 (total store order), so a consumer that reads an env word and
then the block sees the block the producer wrote before the word.  Only the
stage-less ring, whose producers share one write pointer, takes
``reserve_lock``.  A producer that dies after reserving leaves its stage
invisible, and recovery is a whole-run restart, as in the reference.

Device side.  The DMA thread copies each complete stage from the shared
ring into one of a few pinned staging buffers. It then uploads the buffer
into the stage's slot of ``gpu_buffer`` with an asynchronous copy on
``copy_stream`` and records that slot's upload event. Each upload is
ordered after the consumer's last copy out of the same slot by a per-slot
event; nothing else synchronises it. The consumer's stream waits for
exactly the upload event of its stage, copies the rows out and releases
the slot. Every stream keeps the default priority. Memory that already
exists cannot be pinned here, so the shared ring itself is not pinned.

Producer processes.  ``RingStageSource`` starts them from a forkserver with
this module preloaded: a fresh interpreter that never touched the GPU, so
no HIP or profiler state is inherited, and torch is not re-imported per
producer. Each producer owns a contiguous env range and writes it with one
reservation per stage. It exits when it has streamed its stages. ``close``
asks producers to stop, joins them with a grace period, and terminates
only those still alive after it.

Compact records (no reference counterpart; ``record_format="compact"`` of
the pipelines).  ``CompactRingBuffer`` carries 5 bytes per agent-step (int16
position, uint8 action), per-env episode starts and the starting envs'
goals. ``CompactDMAWorker`` uploads a stage and expands it into the 8- or
13-column rows on the device in one native call (``jl_ring_upload_compact``),
so the consumer reads the same rows as from the row ring.
"""
from __future__ import annotations

import ctypes
import hashlib
import json
import multiprocessing as mp
import platform
import signal
import threading
import time
from pathlib import Path

import numpy as np
import torch

FEATURE_DIM = 8
MAPFGPT_FEATURE_DIM = 13
NUM_ACTIONS = 5
RESET_FLAG_COL = 7
# a producer's back-off while its next slot is still in use
_WAIT_S = 0.0005
# the DMA thread's poll when the next stage is not complete yet: a stage of a
# large ring takes a few hundred microseconds end to end, so a 0.5 ms sleep
# would leave the device idle
_DMA_POLL_S = 0.00005
# how long close() lets producers finish before terminating them
_CLOSE_GRACE_S = 5.0


class RingClosed(Exception):
    """Raised in a producer whose stop event was set while it waited for a
    free stage slot."""


_CONTEXT = None


def _process_context():
    """Start method of producer processes, and the context the rings' locks
    and events come from: a forkserver whose server has imported this
    module.  Producers then fork from a process that never touched the GPU,
    and they start without importing torch again.  Where SIGCHLD or SIGINT
    has a handler installed outside Python (a preloaded profiler library
    does this in every process it starts), the forkserver cannot restore it
    in the processes it forks and they exit at once: producers are then
    spawned as fresh interpreters instead."""
    global _CONTEXT
    if _CONTEXT is None:
        foreign = any(signal.getsignal(s) is None for s in (signal.SIGCHLD, signal.SIGINT))
        if foreign:
            _CONTEXT = mp.get_context("spawn")
        else:
            _CONTEXT = mp.get_context("forkserver")
            _CONTEXT.set_forkserver_preload([__name__])
    return _CONTEXT


class _SharedBlock:
    """A shared-memory torch tensor (it travels to forked and
    forkserver-started processes) with a numpy view made on first use in
    each process."""

    def __init__(self, n: int, dtype: torch.dtype, fill: int = 0):
        self.tensor = torch.full((max(1, n),), fill, dtype=dtype).share_memory_()
        self._view = None

    @property
    def view(self) -> np.ndarray:
        if self._view is None:
            self._view = self.tensor.numpy()
        return self._view

    def __getstate__(self):
        return {"tensor": self.tensor, "_view": None}


class _Word:
    """One int64 word of a shared block, read and written through ``.value``
    like a multiprocessing.Value."""

    def __init__(self, block: _SharedBlock, index: int):
        self._block, self._index = block, index

    @property
    def value(self) -> int:
        return int(self._block.view[self._index])

    @value.setter
    def value(self, v: int) -> None:
        self._block.view[self._index] = v


class _PublishedRows:
    """``shared_reserve_ptr`` of a stage ring: the rows published so far,
    derived from the per-env stage words (read only)."""

    def __init__(self, ring: "RingBuffer"):
        self._ring = ring

    @property
    def value(self) -> int:
        return int(self._ring.env_write_seq.sum()) * self._ring.agents_per_env


# control block words
_W_RESERVE, _W_COMPUTE, _W_ENVS = 0, 1, 2


_TSO_MACHINES = ("x86_64", "amd64")


def _require_total_store_order(machine: str | None = None) -> None:
    """The stage ring publishes an env block with plain stores (rows, then the
    env word) and no fence; only a host that keeps stores in program order
    for other cores (x86-64) makes that a publication."""
    machine = (machine if machine is not None else platform.machine()).lower()
    if machine not in _TSO_MACHINES:
        raise RuntimeError(
            f"the stage ring needs a host with total store order (x86-64) to publish stages without a "
            f"lock; this host is {machine!r}")


class RingBuffer:
    """Shared host ring of ``capacity`` rows x ``feature_dim`` int16.

    With ``num_envs`` and ``agents_per_env`` it is a stage ring: capacity is
    a whole number of stages (num_envs * agents_per_env rows each), every
    write is a whole env block, and a stage becomes visible when every env
    has published it.  Without them rows are appended at a shared write
    pointer and marked ready row by row."""

    def __init__(self, capacity: int, feature_dim: int = FEATURE_DIM, *, num_envs: int | None = None,
                 agents_per_env: int | None = None):
        self.capacity = int(capacity)
        self.feature_dim = int(feature_dim)
        self.num_envs = None if num_envs is None else int(num_envs)
        self.agents_per_env = None if agents_per_env is None else int(agents_per_env)
        self.stage_mode = self.num_envs is not None and self.agents_per_env is not None
        self.stage_rows = self.num_stage_slots = None
        if self.stage_mode:
            _require_total_store_order()
            if self.num_envs <= 0:
                raise ValueError(f"num_envs must be positive, got {self.num_envs}")
            if self.agents_per_env <= 0:
                raise ValueError(f"agents_per_env must be positive, got {self.agents_per_env}")
            self.stage_rows = self.num_envs * self.agents_per_env
            if self.capacity % self.stage_rows:
                raise ValueError(
                    "stage-based ring capacity must be divisible by one frontier batch: "
                    f"capacity={self.capacity}, stage_rows={self.stage_rows}")
            self.num_stage_slots = self.capacity // self.stage_rows
            if self.num_stage_slots <= 0:
                raise ValueError(f"stage-based ring requires at least one stage slot, got capacity={capacity}")
        envs = self.num_envs if self.stage_mode else 0
        slots = self.num_stage_slots if self.stage_mode else 0
        self._ctl = _SharedBlock(_W_ENVS + envs + slots, torch.int64)
        self._tags_at = _W_ENVS + envs
        if slots:
            self._ctl.view[self._tags_at:] = -1
        self._flags = _SharedBlock(self.capacity, torch.uint8)
        self.reserve_lock = _process_context().Lock()
        self.cpu_buffer = self._allocate_host_buffer()

    def _allocate_host_buffer(self) -> torch.Tensor:
        return torch.zeros((self.capacity, self.feature_dim), dtype=torch.int16).share_memory_()

    # ---- protocol fields (views of the shared control block) ----------------
    @property
    def ready_flags(self) -> np.ndarray:
        return self._flags.view[:self.capacity]

    @property
    def shared_compute_ptr(self) -> _Word:
        return _Word(self._ctl, _W_COMPUTE)

    @property
    def shared_reserve_ptr(self):
        return _PublishedRows(self) if self.stage_mode else _Word(self._ctl, _W_RESERVE)

    @property
    def env_write_seq(self):
        return self._ctl.view[_W_ENVS:self._tags_at] if self.stage_mode else None

    @property
    def stage_seq_tags(self):
        return self._ctl.view[self._tags_at:self._tags_at + self.num_stage_slots] if self.stage_mode else None

    @property
    def stage_ready_counts(self):
        """Envs that have published the stage each slot holds (0 for a free slot)."""
        if not self.stage_mode:
            return None
        tags = self.stage_seq_tags.copy()
        done = self.env_write_seq.copy()
        counts = (done[None, :] > tags[:, None]).sum(axis=1)
        counts[tags < 0] = 0
        return counts

    # ---- stage protocol ------------------------------------------------------
    def _stage_row_bounds(self, stage_seq: int, env_id: int | None = None) -> tuple[int, int]:
        if not self.stage_mode:
            raise RuntimeError("stage row bounds are only available in stage mode")
        first = int(stage_seq) % self.num_stage_slots * self.stage_rows
        if env_id is None:
            return first, first + self.stage_rows
        first += int(env_id) * self.agents_per_env
        return first, first + self.agents_per_env

    def _reserve_stage_range(self, env_lo: int, env_hi: int, stop=None) -> tuple[int, int, int]:
        """Wait until the next stage of envs [env_lo, env_hi) (one producer's
        range, kept at one stage) has a free slot and tag the slot with it.
        Returns (stage, first row, end row).  The stage stays invisible until
        every env has published it."""
        words = self.env_write_seq[env_lo:env_hi]
        seq = int(words[0])
        if np.any(words != seq):
            raise ValueError("envs of one producer range are at different stages")
        compute = self.shared_compute_ptr
        while seq - compute.value // self.stage_rows >= self.num_stage_slots:
            if stop is not None and stop.is_set():
                raise RingClosed
            time.sleep(_WAIT_S)
        self.stage_seq_tags[seq % self.num_stage_slots] = seq
        first = self._stage_row_bounds(seq, env_lo)[0]
        return seq, first, first + (env_hi - env_lo) * self.agents_per_env

    def _reserve_stage_block(self, env_id: int) -> tuple[int, int, int]:
        return self._reserve_stage_range(env_id, env_id + 1)

    def _publish_stage_range(self, env_lo: int, env_hi: int, stage_seq: int) -> None:
        """Mark the range's rows ready, then publish the envs' stage (the
        store that makes the block visible comes last)."""
        first = self._stage_row_bounds(stage_seq, env_lo)[0]
        self.ready_flags[first:first + (env_hi - env_lo) * self.agents_per_env] = 1
        self.env_write_seq[env_lo:env_hi] = stage_seq + 1

    def _publish_stage_block(self, env_id: int, stage_seq: int) -> None:
        self._publish_stage_range(env_id, env_id + 1, stage_seq)

    def _check_env_block(self, data: np.ndarray) -> int:
        """The env id of one full env block, or ValueError."""
        if data.ndim != 2 or data.shape[1] != self.feature_dim:
            raise ValueError(f"shape must be [N, {self.feature_dim}] in stage mode, got {data.shape}")
        if data.shape[0] != self.agents_per_env:
            raise ValueError("stage-based ring expects one full env block per write: "
                             f"expected {self.agents_per_env} rows, got {data.shape[0]}")
        env_id = int(data[0, 0])
        if not 0 <= env_id < self.num_envs:
            raise ValueError(f"env_id out of range for stage-based ring: env_id={env_id}, num_envs={self.num_envs}")
        if np.any(data[:, 0] != data[0, 0]):
            raise ValueError("stage-based ring requires every written block to contain a single env_id")
        if np.any(data[:, 1] != np.arange(self.agents_per_env)):
            raise ValueError("stage-based ring expects agent ids to be contiguous 0..agents_per_env-1")
        return env_id

    def write_stage_range(self, env_lo: int, rows: np.ndarray, stop=None) -> tuple[int, int]:
        """Write the blocks of the contiguous envs [env_lo, env_lo + n) of
        their next stage (rows [n * agents_per_env, feature_dim], env-major)
        with one reservation; blocks while their slot is in use.  No
        counterpart in the reference, whose producers write one env block
        per call (``reserve_and_write``)."""
        A = self.agents_per_env
        rows = np.asarray(rows)
        if rows.ndim != 2 or rows.shape[1] != self.feature_dim or rows.shape[0] % A or not rows.shape[0]:
            raise ValueError(f"shape must be [n * {A}, {self.feature_dim}] of whole env blocks, got {rows.shape}")
        n_env = rows.shape[0] // A
        env_lo = int(env_lo)
        if env_lo < 0 or env_lo + n_env > self.num_envs:
            raise ValueError(f"env range out of bounds: [{env_lo}, {env_lo + n_env}) of {self.num_envs}")
        ids = rows[:, :2].reshape(n_env, A, 2).astype(np.int64)
        if np.any(ids[:, :, 0] != np.arange(env_lo, env_lo + n_env)[:, None]):
            raise ValueError("stage-based ring requires every written block to contain a single env_id")
        if np.any(ids[:, :, 1] != np.arange(A)[None, :]):
            raise ValueError("stage-based ring expects agent ids to be contiguous 0..agents_per_env-1")
        return self._write_range(env_lo, n_env, rows, stop)

    def _write_range(self, env_lo: int, n_env: int, rows: np.ndarray, stop=None) -> tuple[int, int]:
        seq, first, end = self._reserve_stage_range(env_lo, env_lo + n_env, stop)
        self.cpu_buffer.numpy()[first:end] = rows.astype(np.int16, copy=False)
        self._publish_stage_range(env_lo, env_lo + n_env, seq)
        return first, end

    def _stage_reserve_and_write(self, data: np.ndarray):
        env_id = self._check_env_block(data)
        return self._write_range(env_id, 1, data)

    # ---- writes --------------------------------------------------------------
    def reserve_and_write(self, data: np.ndarray):
        """Write rows (one whole env block on a stage ring); waits while the
        ring is full.  Returns the (start, end) row indices written (end <
        start when the write wrapped)."""
        if self.stage_mode:
            return self._stage_reserve_and_write(np.asarray(data))
        data = np.asarray(data)
        n = int(data.shape[0])
        if n == 0:
            return (0, 0)
        if n > self.capacity:
            raise ValueError(f"cannot write chunk of size {n} into ring buffer capacity {self.capacity}")
        reserve, compute = _Word(self._ctl, _W_RESERVE), self.shared_compute_ptr
        while True:
            with self.reserve_lock:
                start = reserve.value
                if start + n - compute.value <= self.capacity:
                    reserve.value = start + n
                    break
            time.sleep(_WAIT_S)
        begin = start % self.capacity
        head = min(n, self.capacity - begin)  # rows before the end of the buffer
        host = self.cpu_buffer.numpy()
        rows = data.astype(np.int16, copy=False)
        host[begin:begin + head] = rows[:head]
        host[:n - head] = rows[head:]
        self.ready_flags[begin:begin + head] = 1
        self.ready_flags[:n - head] = 1
        return (begin, (begin + n) % self.capacity or self.capacity)

    # ---- consumer side -------------------------------------------------------
    def is_stage_ready(self, stage_seq: int) -> bool:
        if not self.stage_mode:
            return False
        seq = int(stage_seq)
        return bool(self.stage_seq_tags[seq % self.num_stage_slots] == seq and self.env_write_seq.min() > seq)

    def release_stage(self, stage_seq: int) -> None:
        if not self.stage_mode:
            return
        first, end = self._stage_row_bounds(stage_seq)
        self.ready_flags[first:end] = 0
        self.stage_seq_tags[int(stage_seq) % self.num_stage_slots] = -1

    def scan_ready_range(self, start_ptr: int, max_scan: int) -> int:
        """Rows ready from start_ptr on, counting at most max_scan (and not
        past the end of the buffer)."""
        begin = start_ptr % self.capacity
        window = self.ready_flags[begin:begin + max(0, int(max_scan))]
        gaps = np.flatnonzero(window == 0)
        return int(gaps[0]) if gaps.size else int(window.shape[0])

    def clear_flags(self, start: int, end: int) -> None:
        self.ready_flags[start:end] = 0


# ============================================================================
# DMA worker: shared ring -> pinned staging -> HBM ring
# ============================================================================
class DMAWorker:
    """Moves complete stages (or ready rows) of ``ring_buffer`` into the same
    rows of ``gpu_buffer`` from a background thread."""

    def __init__(self, ring_buffer: RingBuffer, gpu_buffer: torch.Tensor, batch_threshold=4096, device="cuda:0",
                 *, staging_slots: int = 2):
        self.ring_buffer = ring_buffer
        self.gpu_buffer = gpu_buffer
        self.batch_threshold = batch_threshold
        self.device = torch.device(device)
        self.dma_read_ptr = 0
        self._running = False
        self._thread = None
        self.copy_stream = torch.cuda.Stream(device=self.device)
        staging_rows = ring_buffer.stage_rows if ring_buffer.stage_mode else max(1, ring_buffer.capacity // 4)
        self.staging = [torch.empty((staging_rows, ring_buffer.feature_dim), dtype=torch.int16).pin_memory()
                        for _ in range(max(1, int(staging_slots)))]
        self._init_events(len(self.staging))
        # set to a list to collect (bytes, start event, end event) per upload
        self.timing = None
        self.host_seconds = 0.0  # host time moving stages (staging copy + enqueue), waits excluded

    def _init_events(self, staging_slots: int) -> None:
        """Events of the upload protocol, each recorded once on the copy
        stream so that it exists (a wait on it is then a no-op) and its
        handle can be passed to native code."""
        slots = self.ring_buffer.num_stage_slots if self.ring_buffer.stage_mode else 1
        self.dma_event = torch.cuda.Event(enable_timing=False)       # after the latest upload
        self.uploaded = [torch.cuda.Event(enable_timing=False) for _ in range(slots)]   # per HBM slot
        self.consumed = [torch.cuda.Event(enable_timing=False) for _ in range(slots)]   # per HBM slot
        self.staging_events = [torch.cuda.Event(enable_timing=False) for _ in range(staging_slots)]
        for ev in (self.dma_event, *self.uploaded, *self.consumed, *self.staging_events):
            ev.record(self.copy_stream)
        self._next_staging = 0

    def _timing_event(self, stream):
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(stream)
        return ev

    def _upload(self, first: int, end: int, slot: int) -> None:
        """Rows [first, end) of the shared ring -> pinned staging -> the same
        rows of gpu_buffer, after the consumer's last copy out of `slot`."""
        k = self._next_staging
        self._next_staging = (k + 1) % len(self.staging)
        self.staging_events[k].synchronize()  # the buffer's previous upload has left host memory
        t_host = time.perf_counter()
        pinned = self.staging[k][:end - first]
        pinned.copy_(self.ring_buffer.cpu_buffer[first:end])
        stream = self.copy_stream
        with torch.cuda.stream(stream):
            self.consumed[slot].wait(stream)
            start = self._timing_event(stream) if self.timing is not None else None
            self.gpu_buffer[first:end].copy_(pinned, non_blocking=True)
            if start is not None:
                self.timing.append((pinned.numel() * pinned.element_size(), start, self._timing_event(stream)))
            self.staging_events[k].record(stream)
            self.uploaded[slot].record(stream)
            self.dma_event.record(stream)
        self.host_seconds += time.perf_counter() - t_host

    def run_once(self):
        """Move the next complete stage (stage ring) or the next ready rows;
        returns the rows moved as (start, end), or None."""
        ring = self.ring_buffer
        if ring.stage_mode:
            seq = self.dma_read_ptr // ring.stage_rows
            if not ring.is_stage_ready(seq):
                return None
            bounds = ring._stage_row_bounds(seq)
            self._upload(*bounds, seq % ring.num_stage_slots)
            self.dma_read_ptr += ring.stage_rows
            return bounds
        pending = ring.shared_reserve_ptr.value - self.dma_read_ptr
        if pending <= 0:
            return None
        begin = self.dma_read_ptr % ring.capacity
        limit = min(pending, ring.capacity - begin, ring.capacity // 4, self.staging[0].shape[0])
        n = ring.scan_ready_range(self.dma_read_ptr, limit)
        if n <= 0:
            return None
        self._upload(begin, begin + n, 0)
        ring.clear_flags(begin, begin + n)
        self.dma_read_ptr += n
        return (begin, begin + n)

    def mark_slot_consumed(self, stage_seq: int, stream) -> None:
        """Record on the consumer's stream that the stage's rows have been
        copied out of gpu_buffer: the slot's next upload waits for it."""
        self.consumed[int(stage_seq) % len(self.consumed)].record(stream)

    def release_completed_stage(self, stage_seq: int) -> None:
        ring = self.ring_buffer
        if not ring.stage_mode:
            return
        ring.release_stage(stage_seq)
        ring.shared_compute_ptr.value = (int(stage_seq) + 1) * ring.stage_rows

    def start(self):
        self._running = True
        self._thread = threading.Thread(target=self._loop, name="ring-dma", daemon=True)
        self._thread.start()
        return self._thread

    def stop(self):
        self._running = False
        t = self._thread
        if t is not None and t is not threading.current_thread():
            t.join(timeout=5.0)

    def _loop(self):
        while self._running:
            if self.run_once() is None:
                time.sleep(_DMA_POLL_S)


# ============================================================================
# Compact stage ring: 5 bytes per agent and step over the host link
# ============================================================================
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
        self._tracked = {}  # producer side: env -> (goals, history) of its running episode

    def _allocate_host_buffer(self) -> torch.Tensor:
        if not self.stage_mode:
            raise ValueError("a compact ring needs num_envs and agents_per_env")
        return torch.zeros((self.num_stage_slots, self.slot_bytes), dtype=torch.uint8).share_memory_()

    def slot_view(self, stage_seq: int) -> np.ndarray:
        """uint8 view of the host slot of a stage."""
        return self.cpu_buffer[int(stage_seq) % self.num_stage_slots].numpy()

    def write_compact(self, env_lo: int, positions, actions, episode_start, goals=None, stop=None):
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
        starting = starts.astype(bool)
        if starting.any() and (goals is None or np.asarray(goals).shape != (n_env * A, 2)):
            raise ValueError("goals [n*A, 2] are required for envs that start an episode")
        seq, first, end = self._reserve_stage_range(env_lo, env_lo + n_env, stop)
        slot = self.slot_view(seq)
        a0, a1 = env_lo * A, (env_lo + n_env) * A
        slot[4 * a0:4 * a1].view(np.uint16)[:] = pos.astype(np.uint16, copy=False).reshape(-1)
        slot[self.off_actions + a0:self.off_actions + a1] = act
        slot[self.off_starts + env_lo:self.off_starts + env_lo + n_env] = starts
        if starting.any():
            src = np.asarray(goals).astype(np.uint16, copy=False).reshape(n_env, 2 * A)
            dst = slot[self.off_goals + 4 * a0:self.off_goals + 4 * a1].view(np.uint16).reshape(n_env, 2 * A)
            dst[starting] = src[starting]
        self._publish_stage_range(env_lo, env_lo + n_env, seq)
        return (first, end)

    def _stage_reserve_and_write(self, data: np.ndarray):
        """A full env block (the reference producer API), compacted."""
        env_id = self._check_env_block(data)
        rows = data.astype(np.int64)
        flags, moves = rows[:, RESET_FLAG_COL], rows[:, 6]
        if np.any(flags > 1) or np.any(moves > 4):
            raise ValueError("invalid action or refresh flag")
        if np.any(flags != flags[0]):
            raise ValueError("compact records need one refresh flag per env and stage")
        starting = bool(flags[0])
        goals = rows[:, 4:6]
        if starting:
            history = np.full((self.agents_per_env, 5), 5, np.int64)
        else:
            if env_id not in self._tracked:
                raise ValueError("compact records need every env to start an episode first")
            kept_goals, history = self._tracked[env_id]
            if not np.array_equal(goals, kept_goals):
                raise ValueError("compact records need goals that change only at an episode start")
        if self.feature_dim == MAPFGPT_FEATURE_DIM and not np.array_equal(rows[:, 8:13], history):
            raise ValueError("history columns are not the previous actions of the episode")
        out = self.write_compact(env_id, rows[:, 2:4], moves, [int(starting)], goals if starting else None)
        self._tracked[env_id] = (goals, np.concatenate([history[:, 1:], moves[:, None]], axis=1))
        return out

    def write_stage_range(self, env_lo: int, rows: np.ndarray, stop=None) -> tuple[int, int]:
        """Row blocks into a compact ring: compacted one env at a time."""
        A = self.agents_per_env
        rows = np.asarray(rows)
        first = None
        for k in range(rows.shape[0] // A):
            bounds = self.reserve_and_write(rows[k * A:(k + 1) * A])
            first = bounds[0] if first is None else first
        return (first, first + rows.shape[0]) if first is not None else (0, 0)


class CompactDMAWorker(DMAWorker):
    """Moves ready compact stages to the device and expands them there into
    ``gpu_buffer`` rows (the same rows a row ring would deliver).

    Per stage one native call (``jl_ring_upload_compact``, run without the
    interpreter lock) copies the slot's head (positions, actions, start
    flags: 5N + E bytes) and the goal range of the envs that start an
    episode from the shared host ring into a pinned staging buffer, uploads
    them on ``copy_stream``, waits on the device for the consumer's copy out
    of the ring slot's rows, expands the stage into ``gpu_buffer`` (advancing
    the running goals and histories) and records the slot's upload event."""

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
        self.dma_read_ptr = 0
        self._running = False
        self._thread = None
        self._lib = load_library()
        self.copy_stream = torch.cuda.Stream(device=self.device)
        k = max(1, int(staging_slots))
        nbytes = ring_buffer.slot_bytes
        self.staging = [torch.empty(nbytes, dtype=torch.uint8).pin_memory() for _ in range(k)]
        self.device_slots = torch.empty((k, nbytes), dtype=torch.uint8, device=self.device)
        self._init_events(k)
        self.expander = RecordExpander(ring_buffer.num_envs, ring_buffer.agents_per_env, ring_buffer.feature_dim,
                                       self.device)
        self.bytes_uploaded = 0
        self.host_seconds = 0.0  # host time of the native step (staging copy + enqueue), waits included
        self.timing = None
        desc = StageUploadDesc()
        desc.slot_bytes = nbytes
        desc.records = self.expander._desc  # sizes, running goals and histories (a copy of the struct)
        self._desc = desc
        self._host_slots = [ring_buffer.cpu_buffer[j].data_ptr() for j in range(ring_buffer.num_stage_slots)]
        self._row_slots = [gpu_buffer[ring_buffer._stage_row_bounds(j)[0]].data_ptr()
                           for j in range(ring_buffer.num_stage_slots)]

    def _upload(self, first: int, end: int, slot: int) -> None:
        from ._abi import check

        t_host = time.perf_counter()
        k = self._next_staging
        self._next_staging = (k + 1) % len(self.staging)
        d = self._desc
        d.host_slot = self._host_slots[slot]
        d.staging = self.staging[k].data_ptr()
        d.device_slot = self.device_slots[k].data_ptr()
        d.staging_free = self.staging_events[k].cuda_event
        d.rows_free = self.consumed[slot].cuda_event
        d.done = self.uploaded[slot].cuda_event
        d.records.rows = self._row_slots[slot]
        start = self._timing_event(self.copy_stream) if self.timing is not None else None
        check(self._lib.jl_ring_upload_compact(ctypes.byref(d), self.copy_stream.cuda_stream), "compact stage upload")
        if start is not None:
            self.timing.append((d.bytes_uploaded, start, self._timing_event(self.copy_stream)))
        self.dma_event.record(self.copy_stream)
        self.bytes_uploaded += d.bytes_uploaded
        self.host_seconds += time.perf_counter() - t_host


# ============================================================================
# Consumers
# ============================================================================
class GPUComputeHandler:
    """MAGAT stage refresh (expert_running.py:537-551): energy fields of the
    agents whose goal was reset, then the compact state of every agent."""

    def __init__(self, simulator):
        self.simulator = simulator

    def filter_reset_agents(self, full_batch: torch.Tensor) -> torch.Tensor:
        return full_batch[full_batch[:, RESET_FLAG_COL].ne(0)]

    def process_batch(self, full_batch: torch.Tensor, agents_to_update: torch.Tensor):
        count = int(agents_to_update.shape[0])
        if count:
            self.simulator.update_derived_state(agents_to_update, count)
        self.simulator.refresh_compact_state_from_raw_batch(full_batch)


class ExtremeMAPFPipeline:
    """Ring + DMA + stage consumer for a MAGAT simulator (expert_running.py:602-808).

    ``initialize`` reads the env layout from the simulator's ``pyg_ptr``
    once (uniform env blocks make it a stage ring); each ``train_step``
    takes the next complete stage, if any, refreshes the simulator from it
    and hands it to the runtime or model."""

    def __init__(self, simulator, capacity=16384 * 128, batch_threshold=16384, feature_dim=FEATURE_DIM,
                 device="cuda:0", *, record_format: str = "rows"):
        if record_format not in ("rows", "compact"):
            raise ValueError(f"record_format must be 'rows' or 'compact', got {record_format!r}")
        self.cuda_simulator = simulator
        self.capacity = capacity
        self.batch_threshold = batch_threshold
        self.feature_dim = feature_dim
        self.device = torch.device(device)
        self.record_format = record_format
        self.ring_buffer = self.gpu_buffer = self.dma_worker = self.gpu_handler = None
        self.dma_event = self.compute_stream = None
        self.dma_read_ptr = self.compute_ptr = 0
        self.graph_rows = None
        self.stage_batch_buffer = None
        self.stage_mode = False
        self.agents_per_env = self.num_envs = None
        self._ids = None  # expected (env, agent) ids of a stage, int16 on the device

    def _infer_stage_layout(self) -> tuple[int | None, int | None]:
        """(agents per env, envs) when pyg_ptr splits the batch into equal
        non-empty env blocks, else (None, None)."""
        ptr = getattr(self.cuda_simulator, "pyg_ptr", None)
        if ptr is None or ptr.shape[0] < 2:
            return None, None
        bounds = ptr.tolist()
        sizes = set(np.diff(bounds).tolist())
        if len(sizes) != 1 or min(sizes) <= 0:
            return None, None
        return sizes.pop(), len(bounds) - 1

    def _make_ring(self, feature_dim: int) -> None:
        compact = self.record_format == "compact"
        ring_cls, dma_cls = (CompactRingBuffer, CompactDMAWorker) if compact else (RingBuffer, DMAWorker)
        self.ring_buffer = ring_cls(self.capacity, feature_dim, num_envs=self.num_envs,
                                    agents_per_env=self.agents_per_env)
        self.gpu_buffer = torch.zeros((self.capacity, feature_dim), dtype=torch.int16, device=self.device)
        rows = self.ring_buffer.stage_rows if self.ring_buffer.stage_mode else self.batch_threshold
        self.stage_batch_buffer = torch.empty((rows, feature_dim), dtype=torch.int16, device=self.device)
        self.dma_worker = dma_cls(self.ring_buffer, self.gpu_buffer, self.batch_threshold, str(self.device))
        self.dma_event = self.dma_worker.dma_event
        self.compute_stream = torch.cuda.Stream(device=self.device)

    def initialize(self):
        self.agents_per_env, self.num_envs = self._infer_stage_layout()
        self.stage_mode = self.agents_per_env is not None
        self._make_ring(self.feature_dim)
        self.gpu_handler = GPUComputeHandler(self.cuda_simulator)
        self.graph_rows = int(self.cuda_simulator.pyg_batch.shape[0])
        return self

    def _require_ring(self):
        if self.ring_buffer is None or self.dma_worker is None:
            raise RuntimeError("Pipeline not initialized. Call initialize() first.")

    def reserve_and_write(self, transitions_numpy):
        self._require_ring()
        return self.ring_buffer.reserve_and_write(transitions_numpy)

    def dma_worker_loop(self):
        self._require_ring()
        self.dma_worker.start()

    def _validate_env_aligned_batch(self, raw_batch: torch.Tensor, agents_per_env: int, num_envs: int) -> None:
        """Env-major blocks with agent ids 0..A-1, checked on the device with
        one host synchronisation."""
        if raw_batch.shape[0] != agents_per_env * num_envs:
            raise ValueError("env-aligned batch size mismatch: "
                             f"expected {agents_per_env * num_envs}, got {raw_batch.shape[0]}")
        key = (num_envs, agents_per_env, raw_batch.device)
        if self._ids is None or self._ids[0] != key:
            env = torch.arange(num_envs, device=raw_batch.device).repeat_interleave(agents_per_env)
            agent = torch.arange(agents_per_env, device=raw_batch.device).repeat(num_envs)
            # uint16 ids as the rows store them (int16 bit patterns)
            ids = torch.stack([env, agent], dim=1).to(torch.int32).remainder(65536)
            self._ids = (key, torch.where(ids > 32767, ids - 65536, ids).to(torch.int16))
        wrong = raw_batch[:, :2].ne(self._ids[1]).any(dim=0).tolist()
        if wrong[0]:
            raise ValueError("stage-based frontier batch must be strict env-major with one block per env")
        if wrong[1]:
            raise ValueError("stage-based frontier batch expects agent ids to be contiguous 0..agents_per_env-1")

    def has_env_aligned_batch(self, num_envs: int) -> bool:
        ring = self.ring_buffer
        return bool(ring is not None and ring.stage_mode and ring.is_stage_ready(self.compute_ptr // ring.stage_rows))

    def extract_env_aligned_batch(self, chunk_size: int, agents_per_env: int, num_envs: int) -> torch.Tensor:
        """The next complete stage as a device tensor (``stage_batch_buffer``,
        valid until the next call), or None when it has not arrived in HBM.
        Work on the current stream is ordered after the stage's upload;
        the stage's slot is released to the producers."""
        ring = self.ring_buffer
        if ring is None or not ring.stage_mode:
            return None
        rows = ring.stage_rows
        seq = self.compute_ptr // rows
        if self.dma_worker.dma_read_ptr - self.compute_ptr < rows:
            return None  # not uploaded yet (the DMA thread checked completeness)
        slot = seq % ring.num_stage_slots
        first, end = ring._stage_row_bounds(seq)
        stream = torch.cuda.current_stream(self.gpu_buffer.device)
        self.dma_worker.uploaded[slot].wait(stream)
        out = self.stage_batch_buffer[:rows]
        out.copy_(self.gpu_buffer[first:end], non_blocking=True)
        self.dma_worker.mark_slot_consumed(seq, stream)
        if not isinstance(self.dma_worker, CompactDMAWorker):
            # the compact expansion writes the ids from the row index itself
            self._validate_env_aligned_batch(out, agents_per_env, num_envs)
        self.compute_ptr += rows
        self.dma_worker.release_completed_stage(seq)
        return out

    def train_step(self, model=None, optimizer=None, runtime=None):
        if self.dma_worker is None or not self.stage_mode:
            return None
        A, E = self.agents_per_env, self.num_envs
        batch = self.extract_env_aligned_batch(A * E, agents_per_env=A, num_envs=E)
        if batch is None:
            return None
        self.gpu_handler.process_batch(batch, self.gpu_handler.filter_reset_agents(batch))
        if runtime is not None:
            return runtime.train_step(self.cuda_simulator, batch)
        if model is None:
            return self.cuda_simulator.pyg_x
        loss = model(self.cuda_simulator.pyg_x)
        if optimizer is not None:
            optimizer.zero_grad(set_to_none=True)
            loss.backward()
            optimizer.step()
        return loss

    def get_stats(self):
        ring = self.ring_buffer
        stats = {
            "capacity": self.capacity,
            "reserve_ptr": ring.shared_reserve_ptr.value if ring is not None else 0,
            "dma_read_ptr": self.dma_worker.dma_read_ptr if self.dma_worker is not None else self.dma_read_ptr,
            "compute_ptr": self.compute_ptr,
        }
        if ring is not None and ring.stage_mode:
            stats["num_stage_slots"] = ring.num_stage_slots
            stats["stage_rows"] = ring.stage_rows
            stats["stage_ready_counts"] = [int(v) for v in ring.stage_ready_counts]
            stats["stage_seq_tags"] = [int(v) for v in ring.stage_seq_tags]
            stats["env_write_stage"] = [int(v) for v in ring.env_write_seq]
        return stats

    def shutdown(self):
        if getattr(self, "dma_worker", None) is not None:
            self.dma_worker.stop()

    def __del__(self):
        self.shutdown()


class MapfGPTOnlinePipeline(ExtremeMAPFPipeline):
    """13-column stages into a MapfGPTObservationBuilder (mapf_gpt_online.py:97-184)."""

    def __init__(self, builder, runtime, *, capacity: int, batch_threshold: int, device: str = "cuda:0",
                 record_format: str = "rows"):
        super().__init__(builder, capacity=capacity, batch_threshold=batch_threshold,
                         feature_dim=MAPFGPT_FEATURE_DIM, device=device, record_format=record_format)
        self.runtime = runtime

    def initialize(self):
        self.agents_per_env, self.num_envs = self._infer_stage_layout()
        if self.agents_per_env is None:
            raise ValueError("MAPF-GPT builder must expose a non-empty pyg_ptr stage layout")
        stage_rows = self.agents_per_env * self.num_envs
        if self.batch_threshold != stage_rows:
            raise ValueError("MAPF-GPT online pipeline requires one complete frontier per batch: "
                             f"expected {stage_rows}, got {self.batch_threshold}")
        self.stage_mode = True
        self._make_ring(MAPFGPT_FEATURE_DIM)
        self.graph_rows = int(self.cuda_simulator.tokens.shape[0])
        return self

    def consume_once(self, *, capture_stage_hash: bool = False):
        """One stage through ``runtime.train_step`` on the compute stream;
        None when the next stage is not in HBM yet."""
        if self.dma_worker is None:
            raise RuntimeError("Pipeline not initialized. Call initialize() first.")
        with torch.cuda.stream(self.compute_stream):
            stage = self.extract_env_aligned_batch(self.agents_per_env * self.num_envs,
                                                   agents_per_env=self.agents_per_env, num_envs=self.num_envs)
            if stage is None:
                return None
            digest = (hashlib.sha256(stage.cpu().numpy().tobytes()).hexdigest() if capture_stage_hash else None)
            metrics = self.runtime.train_step(self.cuda_simulator, stage)
            if digest is not None:
                metrics["stage_sha256"] = digest
            return metrics


# ============================================================================
# Frozen expert records (archive format of frozen_stage_source.py:23-59)
# ============================================================================
_STAGE_MESSAGES = ("coordinates outside map", "coordinates on obstacles", "duplicate joint positions or goals")


def validate_stage(rows, grids, agents, features):
    """A complete env-major uint16 stage of valid records, as [E, A, F]
    blocks (host_inputs.py:17-36).  The checks run over all envs at once;
    the error reported is the one the reference's env-by-env order meets
    first."""
    rows = np.asarray(rows)
    E = len(grids)
    if rows.dtype != np.uint16 or rows.shape != (E * agents, features):
        raise ValueError("stage must contain complete uint16 environment-major records")
    blocks = rows.reshape(E, agents, features)
    if np.any(blocks[:, :, 0] != np.arange(E)[:, None]):
        raise ValueError("stage environment order mismatch")
    if np.any(blocks[:, :, 1] != np.arange(agents)[None, :]):
        raise ValueError("stage agent order mismatch")
    if np.any(rows[:, 6] > 4) or np.any(rows[:, 7] > 1):
        raise ValueError("invalid action or refresh flag")
    # errors[e, k, c]: env e, k = positions / goals, c = outside / obstacle / duplicate
    errors = np.zeros((E, 2, 3), bool)
    shapes = {np.shape(g) for g in grids}
    if len(shapes) == 1:
        grid = np.asarray(grids)
        W, H = grid.shape[1:]
        for k, col in enumerate((2, 4)):
            x = blocks[:, :, col].astype(np.int64)
            y = blocks[:, :, col + 1].astype(np.int64)
            outside = (x >= W) | (y >= H)
            errors[:, k, 0] = outside.any(axis=1)
            env = np.broadcast_to(np.arange(E)[:, None], x.shape)
            inside = ~outside
            blocked = np.zeros_like(outside)
            blocked[inside] = grid[env[inside], x[inside], y[inside]] != 0
            errors[:, k, 1] = blocked.any(axis=1)
            cells = np.sort(x * (H + 1) + y, axis=1)  # distinct within an env iff no equal neighbours
            errors[:, k, 2] = (cells[:, 1:] == cells[:, :-1]).any(axis=1)
    else:
        for e, grid in enumerate(grids):
            grid = np.asarray(grid)
            for k, col in enumerate((2, 4)):
                xy = blocks[e, :, col:col + 2].astype(np.int64)
                outside = (xy[:, 0] >= grid.shape[0]) | (xy[:, 1] >= grid.shape[1])
                errors[e, k, 0] = outside.any()
                errors[e, k, 1] = not outside.any() and bool(grid[xy[:, 0], xy[:, 1]].any())
                errors[e, k, 2] = len(np.unique(xy, axis=0)) != agents
    # the reference stops at an env's positions' first error (outside map
    # before obstacles before duplicates), then its goals, then the next env
    hit = np.flatnonzero(errors.reshape(E * 2, 3).any(axis=1))
    if hit.size:
        kind = int(np.argmax(errors.reshape(E * 2, 3)[hit[0]]))
        raise ValueError(_STAGE_MESSAGES[kind])
    return blocks


def sha256_file(path):
    digest = hashlib.sha256()
    with open(path, "rb") as f:
        while chunk := f.read(1 << 20):
            digest.update(chunk)
    return digest.hexdigest()


def save_records(output, *, backend, grids, stages, metadata):
    """Write grids.npy, stages.npy and a manifest.json with their sha256
    (frozen_stage_source.py:23-42); every stage is validated first."""
    out = Path(output)
    out.mkdir(parents=True, exist_ok=False)
    stages = np.asarray(stages)
    if not np.issubdtype(stages.dtype, np.integer) or stages.size and (stages.min() < 0 or stages.max() > 65535):
        raise ValueError("records must contain uint16-representable integers")
    stages = stages.astype(np.uint16)
    features = FEATURE_DIM if backend == "magat" else MAPFGPT_FEATURE_DIM
    if stages.ndim != 3 or len(stages) == 0 or stages.shape[1] % len(grids):
        raise ValueError("invalid stage archive")
    agents = stages.shape[1] // len(grids)
    for stage in stages:
        validate_stage(stage, grids, agents, features)
    np.save(out / "grids.npy", np.asarray(grids, dtype=np.uint8), allow_pickle=False)
    np.save(out / "stages.npy", stages, allow_pickle=False)
    manifest = {
        "schema_version": 1, "backend": backend, "agents": agents, "stages": len(stages), "features": features,
        "metadata": metadata,
        "hashes": {name: sha256_file(out / name) for name in ("grids.npy", "stages.npy")},
    }
    (out / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n")
    return manifest


def load_records(root):
    """(manifest, grids, memory-mapped stages) of an archive whose hashes,
    shapes and stages check out (frozen_stage_source.py:45-59)."""
    root = Path(root)
    manifest = json.loads((root / "manifest.json").read_text())
    hashes = manifest.get("hashes", {})
    if manifest.get("schema_version") != 1 or set(hashes) != {"grids.npy", "stages.npy"}:
        raise ValueError("unsupported or incomplete record manifest")
    for name, want in hashes.items():
        if sha256_file(root / name) != want:
            raise ValueError(f"record hash mismatch: {name}")
    grids = np.load(root / "grids.npy", allow_pickle=False)
    stages = np.load(root / "stages.npy", mmap_mode="r", allow_pickle=False)
    if stages.shape != (manifest["stages"], len(grids) * manifest["agents"], manifest["features"]):
        raise ValueError("record shape differs from manifest")
    for stage in stages:
        validate_stage(stage, grids, manifest["agents"], manifest["features"])
    return manifest, grids, stages


# ============================================================================
# Producer processes streaming frozen records (frozen_stage_source.py:105-156)
# ============================================================================
def _is_compact(records) -> bool:
    from .records import is_compact_archive

    return is_compact_archive(records)


def _stream_records(worker, env_range, ring, config, records, ready, go, stop, finished):
    """Body of one producer process: open its share of the archive, report
    ready, wait for go, then write envs [lo, hi) of every stage with one
    reservation per stage, and mark itself finished."""
    lo, hi = env_range
    A, steps = config["num_agents"], config["num_steps"]
    try:
        if isinstance(ring, CompactRingBuffer) and _is_compact(records):
            from .records import CompactRecords

            rec = CompactRecords(**{name: np.load(Path(records) / f"{name}.npy", mmap_mode="r", allow_pickle=False)
                                    for name in ("positions", "actions", "episode_starts", "goals")})
            goals = np.zeros(((hi - lo) * A, 2), np.uint16)
            ready.release()
            go.wait()
            for s in range(min(steps, rec.num_stages)):
                if stop.is_set():
                    return
                starts = np.asarray(rec.episode_starts[s, lo:hi])
                for k in np.flatnonzero(starts):
                    goals[k * A:(k + 1) * A] = rec.env_goals(s, lo + int(k))
                ring.write_compact(lo, rec.positions[s, lo * A:hi * A], rec.actions[s, lo * A:hi * A], starts,
                                   goals if starts.any() else None, stop=stop)
        else:
            stages = np.load(Path(records) / "stages.npy", mmap_mode="r", allow_pickle=False)
            ready.release()
            go.wait()
            for s in range(min(steps, len(stages))):
                if stop.is_set():
                    return
                ring.write_stage_range(lo, stages[s, lo * A:hi * A], stop=stop)
        finished[worker] = 1
    except RingClosed:
        return


class RingStageSource:
    """Producer processes streaming frozen records into a stage ring
    (frozen_stage_source.py:105-156).

    By default one process per env, as in the reference; ``workers`` (an
    addition) runs that many processes instead, each owning a contiguous env
    range, for archives with more envs than host cores.  Compact archives
    (records.py) stream into a ``CompactRingBuffer``.  ``check`` raises when
    a producer has exited without finishing its stages."""

    def __init__(self, ring, backend, config, *, records=None, timeout=120, workers=None):
        if records is None:
            raise NotImplementedError("live expert producers (LaCAM + POGEMA) are not part of this build")
        if _is_compact(records) and not isinstance(ring, CompactRingBuffer):
            raise ValueError("compact records stream through a CompactRingBuffer (record_format='compact')")
        self.ring, self.backend, self.timeout = ring, backend, timeout
        self.count = config["num_steps"]
        self.seq = 0
        n_env = len(config["map_names"])
        n_proc = n_env if workers is None else max(1, min(int(workers), n_env))
        ranges = [(w * n_env // n_proc, (w + 1) * n_env // n_proc) for w in range(n_proc)]
        ctx = _process_context()
        self.go, self.stop = ctx.Event(), ctx.Event()
        self._ready = ctx.Semaphore(0)
        self._finished = ctx.RawArray("b", n_proc)
        self.processes = [
            ctx.Process(target=_stream_records, name=f"ring-producer-{w}",
                        args=(w, r, ring, config, str(records), self._ready, self.go, self.stop, self._finished),
                        daemon=True)
            for w, r in enumerate(ranges)
        ]
        try:
            for p in self.processes:
                p.start()
            deadline = time.monotonic() + timeout
            for _ in self.processes:
                while not self._ready.acquire(timeout=0.01):
                    self.check()
                    if time.monotonic() > deadline:
                        raise TimeoutError("expert initialization timeout")
        except BaseException:
            self.close()
            raise

    def check(self):
        """RuntimeError when a producer exited before finishing its stages."""
        codes = [p.exitcode for p in self.processes]
        if any(c is not None and (c != 0 or not self._finished[w]) for w, c in enumerate(codes)):
            raise RuntimeError(f"expert process exited: {codes}")

    def start(self):
        self.go.set()

    def next_rows(self):
        """Host copy of the next complete stage (a CPU consumer of the ring)."""
        if isinstance(self.ring, CompactRingBuffer):
            raise RuntimeError("compact stages are expanded on the device: consume them through the pipeline")
        if self.seq >= self.count:
            raise StopIteration
        deadline = time.monotonic() + self.timeout
        while not self.ring.is_stage_ready(self.seq):
            self.check()
            if time.monotonic() > deadline:
                raise TimeoutError("expert failed to publish a complete stage")
            time.sleep(_WAIT_S)
        first, end = self.ring._stage_row_bounds(self.seq)
        stage = self.ring.cpu_buffer[first:end].numpy().view(np.uint16).copy()
        self.ring.release_stage(self.seq)
        self.seq += 1
        self.ring.shared_compute_ptr.value = self.seq * self.ring.stage_rows
        return stage

    def close(self, grace: float = _CLOSE_GRACE_S):
        """Ask every producer to stop, give them `grace` seconds to exit, and
        terminate only those still running after it."""
        self.stop.set()
        self.go.set()  # producers still waiting to start see stop at once
        deadline = time.monotonic() + grace
        for p in self.processes:
            if p.pid is not None:
                p.join(max(0.0, deadline - time.monotonic()))
        stragglers = [p for p in self.processes if p.pid is not None and p.is_alive()]
        for p in stragglers:
            p.terminate()
        for p in stragglers:
            p.join(2.0)
            if p.is_alive():
                p.kill()
                p.join()
