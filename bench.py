#!/usr/bin/env python3
"""Resident MAPF-GPT rollout throughput on one MI355X (gfx950).

A step is one pass of the north-star hot path over one batch, in the order
of the reference's resident loop (minimal_p0_mapf_gpt_resident_runner.py
:256-281): build_tokens_from_state (goal-cache refresh + BFS of changed goals
+ 256-token contexts), append_actions, update_actions, step_sim_only
(vertex/swap/chain resolution + standard-MAPF bookkeeping).  Actions are
uniform random {0..4} pre-staged in HBM (C2 of BASELINE.json) instead of a
policy forward, so the timed region is the framework's own work.

Workload (BASELINE.json configs[1] + configs[2], the north-star shape):
1024 envs x 128 agents on 64x64 maps, i.i.d. obstacles p=0.2 with the
largest component kept; inputs resident in HBM before timing.  The first
build (every goal fresh: 131,072 BFS fields) happens in the warmup.

Prints one JSON line with the metric, a `roofline` object for the token
kernel (algorithmic bytes / event-timed duration) and a `cpu_baseline`
object (the Python restatement of the reference's cached CPU builder +
step resolver on this host's cores, oracle/host_builder.py).

`--workload magat` measures BASELINE.json's C4 instead (the MAGAT stateful
step of fixed_magat_plus_runtime.py: step_sim_only -> update_derived_state ->
build_magat_plus_nodes -> finalize_magat_plus_graph, plus update_actions) at
512 envs x 256 agents on 64x64 maps with obstacle density 0.3, with the node
kernel's roofline and the C restatement of the same step as CPU baseline.

`--workload ring` streams C5-sized frozen records (256 envs x 1024 agents,
256x256 warehouses) from RingStageSource producer processes through the host
ring and the HBM ring into build_tokens, once in the compact format (5 bytes
per agent-step over the host link, rows rebuilt on the device) and once in the
reference's 13-column row format, with the expansion kernel's roofline.

`--workload costtracer` measures the CostTracer RL environment step of the
online-RL tree (update_actions, a CostTracer-mode step, rewards and goal
streams, the distance refresh of changed goals, the 2x11x11 observation, the
horizon reset) at the C2 shape, with the observation kernel's roofline.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import multiprocessing as mp
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_BPS = 8.0e12
# HBM bytes per build launch measured with rocprofv3 --pmc FETCH_SIZE /
# WRITE_SIZE on this workload, scaled by the copy calibration (file header).
TRAFFIC_FILE = ROOT / "profiles" / "build_kernel_pmc_1024x128_64.txt"

MAGAT_TRAFFIC_FILE = ROOT / "profiles" / "magat_nodes_pmc_512x256_64.txt"
C5_TRAFFIC_FILE = ROOT / "profiles" / "tokens_kernel_pmc_256x1024_256.txt"

# Algorithmic bytes per agent: the compulsory reads and writes of each operation.
B_TOKEN_KERNEL = 8 + 10 + 242 + 1024 + 1  # pos+goal, history, 11x11 u16 window, tokens, mask
# The whole build as one launch (maps of at most 4096 cells): split-array
# position and goal, goal-cache read (written only on a change), history,
# window, state row and label written, tokens, mask.
B_BUILD_SINGLE = 8 + 4 + 10 + 242 + 16 + 8 + 1024 + 1
B_STEP_NORTH_STAR = 1385  # step + token build + append + update_actions per agent-step
# MAGAT node pass: state row, bitmaps share, 11x11 u8 window, 676-float row, pos, count
B_MAGAT_NODES = 16 + 4 + 121 + 2704 + 8 + 4


def cpu_baseline(args) -> dict:
    """Python port of the reference CPU path, one stage per worker process."""
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions
    from oracle.host_builder import run_stage_worker

    cores = len(os.sched_getaffinity(0))
    workers = max(1, min(cores, 16))
    jobs = []
    for w in range(workers):
        grids, starts, goals = make_batch(9000 + w, args.cpu_envs, args.map, args.map, args.agents)
        acts = random_actions(np.random.default_rng(w), args.cpu_steps, args.cpu_envs, args.agents)
        jobs.append((grids, starts, goals, acts, args.cpu_steps))
    ctx = mp.get_context("fork")  # before any HIP call in this process
    t1 = run_stage_worker(jobs[0])
    t0 = time.perf_counter()
    with ctx.Pool(workers) as pool:
        results = pool.map(run_stage_worker, jobs)
    wall = time.perf_counter() - t0
    total = sum(n for _, n in results)
    timed = max(t for t, _ in results)
    return {
        "value": total / timed,
        "unit": "agent-steps/s",
        "cores": workers,
        "workers": workers,
        "host_cpus": host_cpu(),
        "kind": "port",
        "value_1core": t1[1] / t1[0],
        "sample": (
            f"{workers} workers x {args.cpu_envs} envs x {args.agents} agents on {args.map}x{args.map} "
            f"p=0.2, {args.cpu_steps} steady-state steps each (goal cache warm): step resolver + "
            f"cached deque-BFS token builder; pool wall {wall:.1f}s"
        ),
    }


# hipEventDisableSystemFence (hip_runtime_api.h): a timing event recorded
# without a system-scope release.  A default event writes back and
# invalidates the caches where it is recorded, which slowed the resident
# loop by about 7 us per step with two events around every build.
HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000
# the timed loops bracket the hot kernel with events on one step in
# EVENT_EVERY only: each event is a packet of its own that the command
# processor takes about 1.7 us to pass between the kernels, so a pair on
# every fourth step cost the resident loop about 0.9 us per step
EVENT_EVERY = 10


def event_slots(steps: int) -> dict:
    """Timed steps that carry the event pair, each mapped to its slot: the
    middle step of every block of EVENT_EVERY timed steps (the middle step of
    the last, shorter block).  Not each block's first step: the region's
    first step follows its opening synchronize and event (torch records a
    default event, which writes back and invalidates the caches), and the
    first builds after the warmup still run slower while the caches fill, so
    samples at the blocks' starts lean toward those."""
    n = (steps + EVENT_EVERY - 1) // EVENT_EVERY
    return {b * EVENT_EVERY + min(EVENT_EVERY, steps - b * EVENT_EVERY) // 2: b for b in range(n)}


class HipEvents:
    """hipEvent_t handles from the process's HIP runtime (torch's libamdhip64),
    timing-only: created with hipEventDisableSystemFence."""

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so.7")
        self.rt.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.rt.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.rt.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self) -> int:
        ev = ctypes.c_void_p()
        rc = self.rt.hipEventCreateWithFlags(ctypes.byref(ev), HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
        return ev.value

    def event(self) -> "HipTimingEvent":
        return HipTimingEvent(self)

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        rc = self.rt.hipEventElapsedTime(ctypes.byref(ms), ctypes.c_void_p(a), ctypes.c_void_p(b))
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)


class HipTimingEvent:
    """A fence-less timing event with torch.cuda.Event's record / elapsed_time."""

    def __init__(self, hip: HipEvents):
        self.hip = hip
        self.ev = hip.create()

    def record(self, stream=None) -> None:
        import torch

        s = stream if stream is not None else torch.cuda.current_stream()
        rc = self.hip.rt.hipEventRecord(ctypes.c_void_p(self.ev), ctypes.c_void_p(s.cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, other: "HipTimingEvent") -> float:
        return self.hip.elapsed_ms(self.ev, other.ev)


def measured_traffic(path: Path = TRAFFIC_FILE) -> int | None:
    """traffic_bytes from a committed PMC summary, or None."""
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes="):
                return int(float(line.split("=", 1)[1]))
    except OSError:
        return None
    return None


def copy_calibration() -> None:
    """Three device copies of 256 MiB: the reference reading for the PMC
    byte counters (FETCH_SIZE / WRITE_SIZE per dispatch of a known size)."""
    import torch

    n = 256 << 20
    a = torch.empty(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"copied 3 x {n} bytes", flush=True)


def load_probe():
    """libjl_bench.so, the benchmark's own library with the HBM streaming
    probe jl_hbm_stream (built beside libjointloom.so by the package's
    build step; not part of the product library)."""
    import torch  # noqa: F401  (torch's HIP runtime is the process's)

    from iclr_2027_jointoom_amd.build import BENCH_OUTPUT

    if not BENCH_OUTPUT.exists():
        raise RuntimeError(f"{BENCH_OUTPUT} is missing: build first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(str(BENCH_OUTPUT))
    lib.jl_hbm_stream.restype = ctypes.c_int32
    lib.jl_hbm_stream.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                  ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
    return lib


def fetch_probe() -> None:
    """Three launches of jl_hbm_stream kind 10 over 256 MiB: one isolated
    16-byte read per 256-byte block (1,048,576 reads), the reference reading
    for the bytes the L2 fetches per read under the FETCH_SIZE counter."""
    import torch

    from iclr_2027_jointoom_amd._abi import check

    lib = load_probe()
    n = 256 << 20
    a = torch.ones(n // 4, dtype=torch.int32, device="cuda")
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    torch.cuda.synchronize()
    for _ in range(3):
        check(lib.jl_hbm_stream(10, a.data_ptr(), None, n, sink.data_ptr(), cus * 4, stream), "fetch probe")
    torch.cuda.synchronize()
    print(f"3 x {n // 256} isolated 16-byte reads", flush=True)


def achievable_bandwidth(reps: int = 10) -> dict:
    """HBM bandwidth a plain streaming kernel of this library reaches on the
    device (jl_hbm_stream: 16-byte non-temporal loads, non-temporal or plain
    stores, grid-stride or chunked, four accesses in flight per thread) over 1 GiB: read only, write only and
    copy (read + write bytes counted), each the best over a few grid sizes of
    the median of `reps` event-timed launches.  The denominator for
    "fraction of achievable" beside the published peak."""
    import torch

    from iclr_2027_jointoom_amd._abi import check

    lib = load_probe()
    n = 1 << 30
    a = torch.ones(n // 4, dtype=torch.int32, device="cuda")
    b = torch.empty_like(a)
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count

    def launch(kind, wgs):
        check(lib.jl_hbm_stream(kind, a.data_ptr(), b.data_ptr(), n, sink.data_ptr(), wgs, stream),
              "HBM streaming probe")

    def med(kind, wgs):
        launch(kind, wgs)
        times = []
        for _ in range(reps):
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            launch(kind, wgs)
            e.record()
            e.synchronize()
            times.append(s.elapsed_time(e) / 1e3)
        return float(np.median(times))

    out = {}
    # kinds (see jl_hbm_stream): grid-stride 0 read, 1/3 write, 2/4 copy;
    # one contiguous chunk per workgroup 5 read, 6/8 write, 7/9 copy;
    # non-temporal stores in 1, 2, 6, 7, plain ones in 3, 4, 8, 9
    plain = (3, 4, 8, 9)
    for kinds, name, nbytes in (((0, 5), "read", n), ((1, 3, 6, 8), "write", n), ((2, 4, 7, 9), "copy", 2 * n)):
        best = None
        for kind in kinds:
            for per_cu in (2, 4, 8, 16, 32):
                t = med(kind, cus * per_cu)
                if best is None or t < best[0]:
                    best = (t, per_cu, kind)
        out[f"{name}_GBps"] = nbytes / best[0] / 1e9
        out[f"{name}_best"] = (f"{best[1]} workgroups per CU, {'chunked' if best[2] >= 5 else 'grid-stride'}, "
                               f"{'plain' if best[2] in plain else 'non-temporal'} stores")
    del a, b, sink
    torch.cuda.empty_cache()
    out["method"] = ("jl_hbm_stream (this library's streaming kernel: 16-byte accesses, 256-thread workgroups), "
                     "1 GiB each; read only, write only, copy (read + write bytes); best over 2-32 workgroups per "
                     "CU, grid-stride or one contiguous chunk per workgroup, and non-temporal or plain stores, "
                     "of the median of 10 event-timed launches")
    return out


def host_cpu() -> dict:
    """This host's CPU as the baseline line reports it."""
    info = {"model": platform.processor() or "unknown", "logical_cpus": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0))}
    try:
        fields = {}
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = line.split(":", 1)
                fields.setdefault(k.strip(), v.strip())
        info["model"] = fields.get("model name", info["model"])
        info["family_model_stepping"] = "/".join(fields.get(k, "?") for k in ("cpu family", "model", "stepping"))
    except OSError:
        pass
    return info


def TokenMLP():
    """Random-init token policy in bf16: the 256 token values of a context ->
    Linear(256, 64) -> ReLU -> Linear(64, 5).  (An embedding-bag front end
    took 9.5 ms per C5 step in torch, 50x the rest of the step.)"""
    import torch

    class _TokenMLP(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.fc1 = torch.nn.Linear(256, 64)
            self.fc2 = torch.nn.Linear(64, 5)

        def forward(self, tokens):
            return self.fc2(torch.relu(self.fc1(tokens.to(torch.bfloat16))))

    return _TokenMLP()


def run_gpu(args) -> dict:
    import torch

    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = args.envs, args.map, args.agents
    print(f"[bench] generating {E} maps {W}x{W}, {A} agents", file=sys.stderr, flush=True)
    grids, starts, goals = make_batch(args.seed, E, W, W, A, kind=args.map_kind)
    dev = torch.device("cuda:0")
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).to(dev)
    horizon = 1 << 30  # no env reaches its horizon inside the run: every step does full work
    sim = ext.GridWorldSimulator(g, A, 0, E * W * W, 20260728, args.task_mode, horizon)
    sim.load_state(
        torch.from_numpy(starts).to(dev),
        torch.from_numpy(goals).to(dev),
        torch.zeros((E, A), dtype=torch.uint8, device=dev),
        torch.zeros(E, dtype=torch.int32, device=dev),
    )
    if args.task_mode == "lifelong":
        # deterministic lifelong goals: per-env lists of the free cells and
        # per-agent candidate start indices (the online-IL tasks' layout)
        rng = np.random.default_rng(args.seed)
        cells_l = [np.argwhere(gr == 0).astype(np.int16) for gr in grids]
        stride = max(len(c) for c in cells_l)
        cells = np.zeros((E, stride, 2), np.int16)
        for e, c in enumerate(cells_l):
            cells[e, :len(c)] = rng.permutation(c)
        counts = np.array([len(c) for c in cells_l], np.int32)
        cand = rng.integers(0, counts.min(), size=(E, A, 8)).astype(np.int32)
        sim.set_goal_candidates(torch.from_numpy(cand).to(dev), torch.from_numpy(cells).to(dev),
                                torch.from_numpy(counts).to(dev))
    builder = ext.MapfGPTObservationBuilder(g, A)
    builder.reset_histories()
    total_steps = args.warmup + args.steps
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    actions = torch.randint(0, 5, (total_steps, E, A), dtype=torch.uint8, device=dev, generator=gen)
    hip = HipEvents()

    policy = None
    if args.policy == "mlp":
        # token contexts feed a random-init small MLP
        # in PyTorch (bf16, 256 -> 64 -> 5 logits), whose argmax is the next action
        torch.manual_seed(args.seed)
        policy = TokenMLP().to(device=dev, dtype=torch.bfloat16).eval()

    def build():
        builder.build_tokens_from_state(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)

    def act(s):
        if policy is None:
            a = actions[s]
        else:
            with torch.inference_mode():
                a = policy(builder.tokens).argmax(-1).to(torch.uint8).view(E, A)
        builder.append_actions(a)
        sim.update_actions(a)
        sim.step_sim_only()

    def eager_step(s):
        build()
        act(s)

    one_step = eager_step
    graph = None

    def prepare_timed_region():
        # The diagnostics check and the event objects of the timed region,
        # done before the last warmup step: the timed region opens right
        # after that step's synchronize, and no event is created inside it
        # (torch creates one at its first record, a host call that delayed
        # the first timed build by about 14 us).
        torch.cuda.synchronize()
        diag = builder.diagnostics.cpu().tolist()
        if any(diag):
            raise RuntimeError(f"builder diagnostics non-zero after warmup: {diag}")
        # one timed step in EVENT_EVERY carries the event pair around its
        # build (event_slots): each event is a packet of its own that the
        # command processor takes about 1.7 us to pass between the kernels
        evs = [(hip.create(), hip.create()) for _ in event_slots(args.steps)]
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()  # torch creates an event at its first record
        end.record()
        return evs, start, end

    print("[bench] warmup (first build refreshes every goal)", file=sys.stderr, flush=True)
    first_build_ms = None
    timed = None
    for s in range(args.warmup):
        if s == args.warmup - 1 and not args.graph:
            timed = prepare_timed_region()
        if s == 0:
            # the first build computes every agent's field: timed on its own
            torch.cuda.synchronize()
            t_first = time.perf_counter()
            build()
            torch.cuda.synchronize()
            first_build_ms = (time.perf_counter() - t_first) * 1e3
            act(s)
        else:
            one_step(s)
    torch.cuda.synchronize()
    if args.graph and policy is not None:
        raise SystemExit("--graph replays build, append, update and step as one graph, so the policy cannot "
                         "run between the build and the append: use --policy random")
    if args.graph:
        from iclr_2027_jointoom_amd.graphs import MapfGPTResidentGraph

        graph = MapfGPTResidentGraph(sim, builder)

        def one_step(s):
            # the replay reads this step's pre-staged actions where they lie
            graph.replay(actions[s])
    if timed is None:
        timed = prepare_timed_region()
    tok_events, start, end = timed
    slots = event_slots(args.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        if graph is None:
            if i in slots:
                builder._desc.token_events[0], builder._desc.token_events[1] = tok_events[slots[i]]
            else:
                builder._desc.token_events[0] = builder._desc.token_events[1] = None
        one_step(args.warmup + i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    builder._desc.token_events[0] = builder._desc.token_events[1] = None
    gpu_ms = start.elapsed_time(end)
    if graph is not None:
        # events cannot be recorded inside the graph: time the token kernel on
        # eager steps after the timed region
        n_ev = min(len(tok_events), 20)
        tok_events = tok_events[:n_ev]
        for i in range(n_ev):
            builder._desc.token_events[0], builder._desc.token_events[1] = tok_events[i]
            eager_step((args.warmup + i) % total_steps)
        torch.cuda.synchronize()
        builder._desc.token_events[0] = builder._desc.token_events[1] = None
    tok_ms = [hip.elapsed_ms(a, b) for a, b in tok_events]
    diag = builder.diagnostics.cpu().tolist()
    if any(diag):
        raise RuntimeError(f"builder diagnostics non-zero: {diag}")

    N = E * A
    ms_per_step = wall * 1000.0 / args.steps
    value = N * args.steps / wall
    tok_avg_s = float(np.mean(tok_ms)) / 1000.0
    # with a single-launch build the event pair brackets the whole build
    single = builder.single_launch
    tok_bytes = (B_BUILD_SINGLE if single else B_TOKEN_KERNEL) * N
    achieved = tok_bytes / tok_avg_s
    return {
        "value": value,
        "ms_per_step": ms_per_step,
        "gpu_ms_per_step": gpu_ms / args.steps,
        "roofline": {
            "bound": "hbm",
            "kernel": f"build_kernel<{W}> (single-launch build)" if single else f"tokens_kernel<{W}>",
            "achieved": achieved / 1e9,
            "peak": PEAK_HBM_BPS / 1e9,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_BPS,
            # committed PMC summaries: the default workload and C5
            "traffic": (measured_traffic() if (E, A, W, args.map_kind) == (1024, 128, 64, "iid")
                        else measured_traffic(C5_TRAFFIC_FILE) if (E, A, W, args.map_kind) == (256, 1024, 256, "warehouse")
                        else None),
            "bytes_per_launch": tok_bytes,
            "avg_launch_us": tok_avg_s * 1e6,
            "timed_launches": len(tok_ms),  # HIP events on one timed step in EVENT_EVERY (event_slots)
        },
        "first_build_ms": first_build_ms,
        "goals_reassigned": int(sim.goal_cursors.sum().item()) if args.task_mode == "lifelong" else None,
        "step_effective_GBps": value * B_STEP_NORTH_STAR / 1e9,
        "step_frac_of_peak": value * B_STEP_NORTH_STAR / PEAK_HBM_BPS,
        "device": torch.cuda.get_device_name(0),
    }


def bfs_bytes(W: int, H: int) -> int:
    """Algorithmic bytes of one refreshed goal's field: the field written
    (uint16 per cell) and the env's obstacle bitmap read."""
    return 2 * W * H + 4 * W * H // 32


def cpu_baseline_fresh(args) -> dict:
    """The cached CPU builder (oracle/host_builder.py) building with every
    goal fresh: a deque BFS per agent, then the per-ego tokenizer."""
    from iclr_2027_jointoom_amd.synthetic import make_batch
    from oracle.host_builder import run_fresh_worker

    workers = max(1, min(len(os.sched_getaffinity(0)), 16))
    jobs = []
    for w in range(workers):
        grids, starts, goals = make_batch(9100 + w, 1, args.map, args.map, args.agents, kind=args.map_kind)
        jobs.append((grids, starts, goals, 2))
    ctx = mp.get_context("fork")  # before any HIP call in this process
    t1 = run_fresh_worker(jobs[0])
    with ctx.Pool(workers) as pool:
        results = pool.map(run_fresh_worker, jobs)
    total = sum(n for _, n in results)
    timed = max(t for t, _ in results)
    return {
        "value": total / timed,
        "unit": "agent-builds/s (every goal fresh)",
        "cores": workers,
        "workers": workers,
        "host_cpus": host_cpu(),
        "kind": "port",
        "value_1core": t1[1] / t1[0],
        "sample": (f"{workers} workers x 1 env x {args.agents} agents on {args.map}x{args.map} {args.map_kind} maps, "
                   f"2 builds each with every goal fresh (deque BFS per agent + per-ego tokenizer)"),
    }


def run_gpu_fresh(args) -> dict:
    """Builds with every goal fresh (C3: all E*A BFS fields, then the tokens),
    each after the goal cache is cleared; the build launch is event-timed."""
    import torch

    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = args.envs, args.map, args.agents
    print(f"[bench] fresh builds: {E} {args.map_kind} maps {W}x{W}, {A} agents", file=sys.stderr, flush=True)
    grids, starts, goals = make_batch(args.seed, E, W, W, A, kind=args.map_kind)
    dev = torch.device("cuda:0")
    g = torch.from_numpy(grids.astype(np.int32)).to(dev)
    ext = profile(W, W)
    builder = ext.MapfGPTObservationBuilder(g, A)
    builder.reset_histories()
    st = [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in
          (starts[..., 0], starts[..., 1], goals[..., 0], goals[..., 1])]
    hip = HipEvents()
    for _ in range(args.warmup):
        builder.goal_cache.fill_(-1)
        builder.build_tokens_from_state(*st)
    torch.cuda.synchronize()
    events = [(hip.create(), hip.create()) for _ in range(args.steps)]
    wall = 0.0
    for i in range(args.steps):
        builder.goal_cache.fill_(-1)  # every goal fresh: all E*A fields are refreshed
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        builder._desc.token_events[0], builder._desc.token_events[1] = events[i]
        builder.build_tokens_from_state(*st)
        torch.cuda.synchronize()
        wall += time.perf_counter() - t0
    builder._desc.token_events[0] = builder._desc.token_events[1] = None
    diag = builder.diagnostics.cpu().tolist()
    if any(diag):
        raise RuntimeError(f"builder diagnostics non-zero: {diag}")
    ms = [hip.elapsed_ms(a, b) for a, b in events]
    build_s = float(np.median(ms)) / 1e3
    N = E * A
    per_agent = bfs_bytes(W, W) + (B_BUILD_SINGLE if builder.single_launch else B_TOKEN_KERNEL)
    return {
        "value": N / build_s,
        "ms_per_build": build_s * 1e3,
        "wall_ms_per_build": wall * 1e3 / args.steps,
        "fields_per_s": N / build_s,
        "roofline": {
            "bound": "hbm",
            "kernel": f"build_kernel<{W}> (single-launch build, every goal fresh)" if builder.single_launch
                      else f"bfs + tokens_kernel<{W}>",
            "achieved": per_agent * N / build_s / 1e9,
            "peak": PEAK_HBM_BPS / 1e9,
            "unit": "GB/s",
            "frac": per_agent * N / build_s / PEAK_HBM_BPS,
            "traffic": None,
            "bytes_per_launch": per_agent * N,
            "bytes_per_agent": per_agent,
            "bfs_bytes_per_field": bfs_bytes(W, W),
            "avg_launch_us": build_s * 1e6,
        },
        "device": torch.cuda.get_device_name(0),
    }


def main_fresh(args) -> int:
    base = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        base = cpu_baseline_fresh(args)
    res = run_gpu_fresh(args)
    line = {
        "metric": "agent-steps/sec incl. obs/token build on 1 GPU; % of HBM roofline",
        "value": res["value"],
        "unit": "agent-builds/s (every goal fresh: BFS field + tokens per agent)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_build"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16/int32 (integer)",
        "data": f"synthetic (seeded {args.map_kind} maps, largest component; distinct starts/goals)",
        "config": {
            "workload": "C3 fresh build: every goal's cost-to-go BFS field + MAPF-GPT tokens",
            "envs": args.envs,
            "agents": args.agents,
            "map": f"{args.map}x{args.map}",
            "map_kind": args.map_kind,
            "fields_per_build": args.envs * args.agents,
        },
        "roofline": res["roofline"],
        "cpu_baseline": base,
        "wall_ms_per_build": res["wall_ms_per_build"],
        "device": res["device"],
    }
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_sampled(args, *, records: bool) -> dict:
    """The host path of the C5 shape on a bounded sample: one env of the
    workload per worker process (256x256 warehouse, its full agent count),
    goal cache warm (filled before timing).  records=False: resident steps
    (step resolver + cached token builder); records=True: the frozen-record
    consumer, the cached builder over successive stages."""
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions
    from oracle.host_builder import run_stage_build_worker, run_stage_worker

    workers = max(1, min(len(os.sched_getaffinity(0)), 16))
    steps = args.cpu_steps
    jobs = []
    for w in range(workers):
        grids, starts, goals = make_batch(9200 + w, 1, args.map, args.map, args.agents, kind=args.map_kind)
        if records:
            pos = np.stack([np.roll(starts, k, axis=1) for k in range(steps + 1)])  # distinct cells per stage
            jobs.append((grids, pos, goals))
        else:
            acts = random_actions(np.random.default_rng(w), steps, 1, args.agents)
            jobs.append((grids, starts, goals, acts, steps, True))
    fn = run_stage_build_worker if records else run_stage_worker
    ctx = mp.get_context("fork")  # before any HIP call in this process
    t1 = fn(jobs[0])
    with ctx.Pool(workers) as pool:
        results = pool.map(fn, jobs)
    total = sum(n for _, n in results)
    timed = max(t for t, _ in results)
    what = ("cached token builder over successive frozen stages" if records
            else "step resolver + cached token builder (no policy)")
    return {
        "value": total / timed,
        "unit": "agent-steps/s",
        "cores": workers,
        "workers": workers,
        "host_cpus": host_cpu(),
        "kind": "port",
        "value_1core": t1[1] / t1[0],
        "sample": (f"{workers} workers x 1 env x {args.agents} agents on {args.map}x{args.map} {args.map_kind} maps, "
                   f"{steps} timed steps each, goal cache warm: {what}"),
    }


def cpu_baseline_magat(args) -> dict:
    """The C restatement of the stateful MAGAT step, one env per worker."""
    from iclr_2027_jointoom_amd.synthetic import make_batch, random_actions
    from oracle.host_builder import run_magat_worker

    cores = len(os.sched_getaffinity(0))
    workers = max(1, min(cores, 16))
    jobs = []
    for w in range(workers):
        grids, starts, goals = make_batch(7000 + w, 1, args.map, args.map, args.agents, density=0.3)
        acts = random_actions(np.random.default_rng(w), args.cpu_steps, 1, args.agents)
        jobs.append((grids, starts, goals, acts, args.cpu_steps))
    ctx = mp.get_context("fork")  # before any HIP call in this process
    t1 = run_magat_worker(jobs[0])
    t0 = time.perf_counter()
    with ctx.Pool(workers) as pool:
        results = pool.map(run_magat_worker, jobs)
    wall = time.perf_counter() - t0
    total = sum(n for _, n in results)
    timed = max(t for t, _ in results)
    return {
        "value": total / timed,
        "unit": "agent-steps/s",
        "cores": workers,
        "workers": workers,
        "host_cpus": host_cpu(),
        "kind": "port",
        "value_1core": t1[1] / t1[0],
        "sample": (
            f"{workers} workers x 1 env x {args.agents} agents on {args.map}x{args.map} p=0.3, "
            f"{args.cpu_steps} steps each: C restatement (oracle/jl_oracle.c) of step, occupancy, "
            f"nodes and edges; pool wall {wall:.1f}s"
        ),
    }


def run_gpu_magat(args) -> dict:
    import torch

    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, A, W = args.envs, args.agents, args.map
    print(f"[bench] generating {E} maps {W}x{W} (p=0.3), {A} agents", file=sys.stderr, flush=True)
    grids, starts, goals = make_batch(args.seed, E, W, W, A, density=0.3)
    dev = torch.device("cuda:0")
    g = torch.from_numpy(grids.astype(np.int32)).to(dev)
    sim = profile(W, W).GridWorldSimulator(g, A, 3, E * W * W, 20260728, "standard_mapf", 1 << 30)
    sim.load_state(
        torch.from_numpy(starts).to(dev),
        torch.from_numpy(goals).to(dev),
        torch.zeros((E, A), dtype=torch.uint8, device=dev),
        torch.zeros(E, dtype=torch.int32, device=dev),
    )
    total_steps = args.warmup + args.steps
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    actions = torch.randint(0, 5, (total_steps, E, A), dtype=torch.uint8, device=dev, generator=gen)

    def one_step(s, ev=None):
        sim.update_actions(actions[s])
        sim.step_sim_only()
        sim.update_derived_state()
        if ev is not None:
            ev[0].record()
        sim.build_magat_plus_nodes()
        if ev is not None:
            ev[1].record()
        sim.finalize_magat_plus_graph()
        if ev is not None:
            ev[2].record()

    print("[bench] warmup (the first step builds every energy field)", file=sys.stderr, flush=True)
    for s in range(args.warmup):
        one_step(s)
    torch.cuda.synchronize()
    graph = None
    if args.graph:
        from iclr_2027_jointoom_amd.graphs import MagatStatefulGraph

        graph = MagatStatefulGraph(sim)
    # all kernels run on torch's current stream, so events recorded there bracket the node pass
    hip = HipEvents()
    slots = event_slots(args.steps)
    node_events = [tuple(hip.event() for _ in range(3)) for _ in slots]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        if graph is None:
            one_step(args.warmup + i, node_events[slots[i]] if i in slots else None)
        else:
            graph.replay(actions[args.warmup + i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    if graph is not None:
        # events cannot be recorded inside the graph: time the node pass on
        # eager steps after the timed region
        node_events = node_events[:20]
        for i, ev in enumerate(node_events):
            one_step((args.warmup + i) % total_steps, ev)
        torch.cuda.synchronize()
    node_ms = [a.elapsed_time(b) for a, b, _ in node_events]
    # the graph pass: env scan + edge writer (finalize_magat_plus_graph)
    graph_ms = [b.elapsed_time(c) for _, b, c in node_events]
    N = E * A
    value = N * args.steps / wall
    node_s = float(np.mean(node_ms)) / 1000.0
    node_bytes = B_MAGAT_NODES * N
    achieved = node_bytes / node_s
    return {
        "value": value,
        "ms_per_step": wall * 1000.0 / args.steps,
        "roofline": {
            "bound": "hbm",
            "kernel": f"nodes_kernel<{W}>",
            "achieved": achieved / 1e9,
            "peak": PEAK_HBM_BPS / 1e9,
            "unit": "GB/s",
            "frac": achieved / PEAK_HBM_BPS,
            "traffic": measured_traffic(MAGAT_TRAFFIC_FILE) if (E, A, W) == (512, 256, 64) else None,
            "bytes_per_launch": node_bytes,
            "avg_launch_us": node_s * 1e6,
            "timed_launches": len(node_ms),  # HIP events on one timed step in EVENT_EVERY (event_slots)
        },
        "edges_per_step": int(sim.pyg_num_edges.item()),
        "graph_us": float(np.mean(graph_ms)) * 1e3,
        "device": torch.cuda.get_device_name(0),
    }


def main_magat(args) -> int:
    base = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        base = cpu_baseline_magat(args)
    res = run_gpu_magat(args)
    line = {
        "metric": "agent-steps/sec incl. obs/token build on 1 GPU; % of HBM roofline",
        "value": res["value"],
        "unit": "agent-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16/int32 (integer) + float32 node features",
        "data": "synthetic (seeded i.i.d. maps p=0.3, largest component; distinct starts/goals; uniform random actions)",
        "config": {
            "workload": "MAGAT stateful step + FOV/graph build (C4)",
            "launch": "hip-graph replay" if args.graph else "eager",
            "envs": args.envs,
            "agents": args.agents,
            "map": f"{args.map}x{args.map}",
            "task_mode": "standard_mapf",
        },
        "roofline": res["roofline"],
        "cpu_baseline": base,
        "edges_per_step": res["edges_per_step"],
        "graph_us": res["graph_us"],
        "device": res["device"],
    }
    print(json.dumps(line), flush=True)
    return 0


def _ring_row_stages(positions, actions, goals, E: int, A: int) -> np.ndarray:
    """Full 13-column rows of one episode per env starting at stage 0 (the rows
    mapf_gpt_expert_worker_loop writes, mapf_gpt_online.py:215-258)."""
    S, N = actions.shape
    rows = np.empty((S, N, 13), np.uint16)
    rows[:, :, 0] = np.repeat(np.arange(E, dtype=np.uint16), A)[None]
    rows[:, :, 1] = np.tile(np.arange(A, dtype=np.uint16), E)[None]
    rows[:, :, 2:4] = positions
    rows[:, :, 4:6] = goals.reshape(N, 2)[None]
    rows[:, :, 6] = actions
    rows[:, :, 7] = 0
    rows[0, :, 7] = 1
    for k in range(5):  # history slot k at stage s holds the action of stage s - 5 + k
        lag = 5 - k
        rows[:lag, :, 8 + k] = 5
        rows[lag:, :, 8 + k] = actions[:S - lag]
    return rows


def run_gpu_ring(args) -> dict:
    """Frozen records -> RingStageSource producers -> host ring -> HBM ring ->
    build_tokens, for the compact format and the reference's row format."""
    import shutil
    import tempfile

    import torch

    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.records import CompactRecords, write_compact_records
    from iclr_2027_jointoom_amd.ring import MapfGPTOnlinePipeline, RingStageSource, save_records
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = args.envs, args.map, args.agents
    N = E * A
    S = args.warmup + args.steps
    print(f"[bench] ring: generating {E} maps {W}x{W}, {A} agents, {S} stages", file=sys.stderr, flush=True)
    grids, starts, goals = make_batch(args.seed, E, W, W, A, kind=args.map_kind)
    rng = np.random.default_rng(args.seed)
    positions = np.empty((S, N, 2), np.uint16)
    pos = starts.astype(np.uint16)
    for s in range(S):
        positions[s] = pos.reshape(N, 2)
        pos = np.roll(pos, 1, axis=1)  # distinct free cells at every stage
    actions = rng.integers(0, 5, size=(S, N)).astype(np.uint8)
    episode_starts = np.zeros((S, E), np.uint8)
    episode_starts[0] = 1
    tmp = Path(tempfile.mkdtemp(prefix="jl_ring_", dir=os.environ.get("TMPDIR", "/tmp")))
    archives = {}
    try:
        rec = CompactRecords(positions, actions, episode_starts, goals.astype(np.uint16))
        write_compact_records(tmp / "compact", backend="mapf_gpt", grids=grids, records=rec, metadata={})
        archives["compact"] = tmp / "compact"
        if not args.ring_compact_only:
            save_records(tmp / "rows", backend="mapf_gpt", grids=grids,
                         stages=_ring_row_stages(positions, actions, goals, E, A), metadata={})
            archives["rows"] = tmp / "rows"
        dev = torch.device("cuda:0")
        g = torch.from_numpy(grids.astype(np.int32)).to(dev)
        ext = profile(W, W)
        hip = HipEvents()
        config = {"num_agents": A, "num_steps": S, "map_names": [f"env{e}" for e in range(E)]}
        out = {}
        for fmt, path in archives.items():
            builder = ext.MapfGPTObservationBuilder(g, A)
            slots = event_slots(args.steps)
            tok_events = [(hip.create(), hip.create()) for _ in slots]

            class _Build:
                n = 0

                def train_step(self, b, raw):
                    i = self.n - args.warmup
                    if i in slots:
                        b._desc.token_events[0], b._desc.token_events[1] = tok_events[slots[i]]
                    else:
                        b._desc.token_events[0] = b._desc.token_events[1] = None
                    b.build_tokens(raw)
                    self.n += 1
                    return {}

            runtime = _Build()
            pipe = MapfGPTOnlinePipeline(builder, runtime, capacity=args.ring_slots * N, batch_threshold=N,
                                         device=str(dev), record_format=fmt).initialize()
            pipe.dma_worker.timing = []
            src = RingStageSource(pipe.ring_buffer, "mapf_gpt", config, records=path, timeout=600,
                                  workers=args.ring_workers)
            print(f"[bench] ring {fmt}: {len(src.processes)} producer processes", file=sys.stderr, flush=True)
            try:
                src.start()
                pipe.dma_worker_loop()
                done = 0
                t0 = None
                busy = 0.0
                while done < S:
                    if done == args.warmup and t0 is None:
                        torch.cuda.synchronize()
                        t0 = time.perf_counter()
                        dma_host0 = pipe.dma_worker.host_seconds
                    tc = time.perf_counter()
                    if pipe.consume_once() is None:
                        src.check()
                        time.sleep(0.00005)
                    else:
                        done += 1
                        if t0 is not None:
                            busy += time.perf_counter() - tc
                torch.cuda.synchronize()
                wall = time.perf_counter() - t0
                dma_host = pipe.dma_worker.host_seconds - dma_host0
            finally:
                pipe.shutdown()
                src.close()
            builder._desc.token_events[0] = builder._desc.token_events[1] = None
            diag = builder.diagnostics.cpu().tolist()
            if any(diag):
                raise RuntimeError(f"builder diagnostics non-zero: {diag}")
            timing = pipe.dma_worker.timing[args.warmup:]
            up_bytes = float(np.mean([t[0] for t in timing]))
            # rows: the upload (the compact step's events also span its device-side
            # wait for the consumer, so the compact line reports bytes only)
            up_s = float(np.mean([t[1].elapsed_time(t[2]) for t in timing])) / 1e3 if fmt == "rows" else None
            res = {
                "value": N * args.steps / wall,
                "ms_per_stage": wall * 1e3 / args.steps,
                "host_link_bytes_per_stage": up_bytes,
                "host_link_bytes_per_agent_step": up_bytes / N,
                "upload_us_per_stage": up_s * 1e6 if up_s else None,
                "upload_GBps": up_bytes / up_s / 1e9 if up_s else None,
                "token_us": float(np.mean([hip.elapsed_ms(a, b) for a, b in tok_events])) * 1e3,
                "consumer_host_us_per_stage": busy * 1e6 / args.steps,
                "dma_host_us_per_stage": dma_host * 1e6 / args.steps,
                "producers": len(src.processes),
            }
            if fmt == "compact":
                res["expand_us"] = time_expansion(rec, E, A, dev)
            out[fmt] = res
            print(f"[bench] ring {fmt}: {json.dumps(res)}", file=sys.stderr, flush=True)
            del pipe, builder, runtime
            torch.cuda.empty_cache()
        out["device"] = torch.cuda.get_device_name(0)
        return out
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def time_expansion(rec, E: int, A: int, dev, reps: int = 50) -> float:
    """Average duration (us, HIP events on the current stream) of
    jl_expand_records over one steady-state stage of the archive."""
    import torch

    from iclr_2027_jointoom_amd.records import RecordExpander

    N = E * A
    exp = RecordExpander(E, A, 13, dev)
    pos = torch.from_numpy(np.ascontiguousarray(rec.positions[1]).view(np.int16)).to(dev)
    act = torch.from_numpy(np.ascontiguousarray(rec.actions[1])).to(dev)
    first = torch.ones(E, dtype=torch.uint8, device=dev)
    cont = torch.zeros(E, dtype=torch.uint8, device=dev)
    goals = torch.from_numpy(np.ascontiguousarray(rec.goals).reshape(N, 2).view(np.int16)).to(dev)
    rows = torch.empty((N, 13), dtype=torch.int16, device=dev)
    exp.expand(pos, act, first, goals, rows)
    # the launches are captured into a HIP graph and replayed between one
    # event pair: separate launches from the host leave gaps longer than this
    # few-microsecond kernel
    ptrs = (pos.data_ptr(), act.data_ptr(), cont.data_ptr(), goals.data_ptr(), rows.data_ptr())
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.graph(graph, stream=side):
        for _ in range(reps):
            exp.expand_ptrs(*ptrs, side.cuda_stream)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph.replay()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


# expansion of one steady-state 13-column stage per agent: positions + action
# read (5), running goal read (4), history read + write (8 + 8), row write (26)
B_EXPAND_13 = 5 + 4 + 8 + 8 + 26


def main_ring(args) -> int:
    base = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        base = cpu_baseline_sampled(args, records=True)
    res = run_gpu_ring(args)
    c = res["compact"]
    N = args.envs * args.agents
    tok_s = c["token_us"] / 1e6
    exp_s = c["expand_us"] / 1e6
    line = {
        "metric": "agent-steps/sec incl. obs/token build on 1 GPU; % of HBM roofline",
        "value": c["value"],
        "unit": "agent-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": c["ms_per_stage"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16/int32 (integer)",
        "data": "synthetic frozen records (seeded warehouse maps, distinct positions and goals, uniform actions)",
        "config": {
            "workload": "frozen records streamed through the HBM ring into build_tokens (C5 ring)",
            "record_format": "compact (5 B per agent-step, rows rebuilt on the device)",
            "envs": args.envs,
            "agents": args.agents,
            "map": f"{args.map}x{args.map}",
            "producers": c["producers"],
            "ring_slots": args.ring_slots,
        },
        # the dominant kernel of a stage is the token pass; the expansion that
        # replaces the 26-byte rows on the link is reported beside it
        "roofline": {
            "bound": "hbm",
            "kernel": f"tokens_kernel<{args.map}>",
            "achieved": B_TOKEN_KERNEL * N / tok_s / 1e9,
            "peak": PEAK_HBM_BPS / 1e9,
            "unit": "GB/s",
            "frac": B_TOKEN_KERNEL * N / tok_s / PEAK_HBM_BPS,
            "traffic": None,
            "bytes_per_launch": B_TOKEN_KERNEL * N,
            "avg_launch_us": c["token_us"],
        },
        "expand_roofline": {
            "kernel": "expand_records_kernel<13>",
            "achieved": B_EXPAND_13 * N / exp_s / 1e9,
            "frac": B_EXPAND_13 * N / exp_s / PEAK_HBM_BPS,
            "bytes_per_launch": B_EXPAND_13 * N,
            "avg_launch_us": c["expand_us"],
        },
        "cpu_baseline": base,
        "compact": c,
        "rows": res.get("rows"),
        "device": res["device"],
    }
    print(json.dumps(line), flush=True)
    return 0


# CostTracer observation per agent: 11x11 uint16 window 242, 242 floats out 968,
# the window's occupancy bits 16, position 4, refresh flag 2, best read+write 8
B_CT_OBSERVE = 242 + 968 + 16 + 4 + 2 + 8


def cpu_baseline_costtracer(args) -> dict:
    """The CostTracer environment loop on the host cores (oracle/costtracer.py:
    C step oracle + numpy observation + C BFS of changed goals), one block of
    envs per worker process, as the reference's CpuPool runs its envs."""
    from iclr_2027_jointoom_amd.synthetic import make_batch
    from oracle.costtracer import run_costtracer_worker

    cores = len(os.sched_getaffinity(0))
    workers = max(1, min(cores, 16))
    jobs = []
    for w in range(workers):
        grids, starts, goals = make_batch(7000 + w, args.cpu_envs, args.map, args.map, args.agents)
        streams = np.stack([np.roll(goals, k + 1, axis=1) for k in range(16)], axis=2).astype(np.int16)
        acts = np.random.default_rng(w).integers(0, 5, (args.cpu_steps, args.cpu_envs, args.agents)).astype(np.uint8)
        jobs.append((grids, starts, goals, streams, acts, args.cpu_steps))
    ctx = mp.get_context("fork")  # before any HIP call in this process
    t1 = run_costtracer_worker(jobs[0])
    with ctx.Pool(workers) as pool:
        results = pool.map(run_costtracer_worker, jobs)
    total = sum(n for _, n in results)
    timed = max(t for t, _ in results)
    return {
        "value": total / timed,
        "unit": "agent-steps/s",
        "cores": workers,
        "workers": workers,
        "host_cpus": host_cpu(),
        "kind": "port",
        "value_1core": t1[1] / t1[0],
        "sample": (f"{workers} workers x {args.cpu_envs} envs x {args.agents} agents on {args.map}x{args.map} "
                   f"p=0.2, {args.cpu_steps} CostTracer steps each (step, reward and goal stream, BFS of "
                   f"changed goals, observation)"),
    }


def run_gpu_costtracer(args) -> dict:
    """The CostTracer environment step of rebuttal/online-rl/implementation/
    environments.py:206-217 (update_actions, step in CostTracer mode, reward
    and goal streams, refresh_distances, observation) plus reset_due."""
    import torch

    from iclr_2027_jointoom_amd import profile
    from iclr_2027_jointoom_amd.synthetic import make_batch

    E, W, A = args.envs, args.map, args.agents
    horizon = args.ct_horizon
    print(f"[bench] costtracer: {E} maps {W}x{W}, {A} agents, horizon {horizon}", file=sys.stderr, flush=True)
    grids, starts, goals = make_batch(args.seed, E, W, W, A, kind=args.map_kind)
    rng = np.random.default_rng(args.seed)
    bank = 2
    bank_pos = np.stack([starts] + [np.stack([s[rng.permutation(A)] for s in starts]) for _ in range(bank - 1)])
    bank_goal = np.stack([goals] + [np.stack([g[rng.permutation(A)] for g in goals]) for _ in range(bank - 1)])
    dev = torch.device("cuda:0")
    K = horizon + 1
    # goal streams: each agent cycles through rolled copies of its env's goal set (free, distinct cells)
    streams = torch.stack([torch.from_numpy(np.stack([np.roll(bank_goal[ep], k + 1, axis=1) for k in range(K)],
                                                     axis=2).astype(np.int16)) for ep in range(bank)]).to(dev)
    ext = profile(W, W)
    g = torch.from_numpy(grids.astype(np.int32)).to(dev)
    sim = ext.GridWorldSimulator(g, A, 0, E * W * W, 3, "costtracer", horizon)
    builder = ext.MapfGPTObservationBuilder(g, A)
    bp = torch.from_numpy(bank_pos.astype(np.int16)).to(dev)
    bg = torch.from_numpy(bank_goal.astype(np.int16)).to(dev)
    episodes = torch.zeros(E, dtype=torch.int32, device=dev)
    stream = streams[0].contiguous()
    cursor = torch.zeros((E, A), dtype=torch.int32, device=dev)
    best = torch.full_like(cursor, -1)
    reward = torch.empty((E, A), device=dev)
    reached = torch.empty_like(reward)
    obs = torch.empty((E, A, 2, 11, 11), device=dev)
    sim.load_state(bp[0], bg[0], torch.zeros((E, A), dtype=torch.uint8, device=dev),
                   torch.zeros(E, dtype=torch.int32, device=dev))
    total = args.warmup + args.steps
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    actions = torch.randint(0, 5, (total, E, A), dtype=torch.uint8, device=dev, generator=gen)

    def observe(ev=None):
        builder.refresh_distances(sim.cur_x, sim.cur_y, sim.goal_x, sim.goal_y)
        if ev is not None:
            ev[0].record()
        ext.costtracer_observe(sim, builder, best, obs)
        if ev is not None:
            ev[1].record()

    def one_step(s, ev=None):
        sim.update_actions(actions[s])
        sim.step_sim_only()
        ext.costtracer_reward_goals(sim, builder, best, stream, cursor, reward, reached)
        observe(ev)
        # envs at the horizon restart from the bank (a no-op launch otherwise);
        # the stream of a restarted env stays the one it had, as the bench
        # keeps every env on its bank's first streams
        ext.costtracer_reset(sim, bp, bg, episodes, cursor, best, episodes, horizon)

    print("[bench] warmup (the first refresh computes every BFS field)", file=sys.stderr, flush=True)
    observe()
    for s in range(args.warmup):
        one_step(s)
    torch.cuda.synchronize()
    if any(builder.diagnostics.cpu().tolist()):
        raise RuntimeError(f"builder diagnostics non-zero: {builder.diagnostics.cpu().tolist()}")
    hip = HipEvents()
    slots = event_slots(args.steps)
    obs_events = [(hip.event(), hip.event()) for _ in slots]
    hits0 = int(cursor.sum().item())
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        one_step(args.warmup + i, obs_events[slots[i]] if i in slots else None)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    obs_s = float(np.mean([a.elapsed_time(b) for a, b in obs_events])) / 1000.0
    N = E * A
    nbytes = B_CT_OBSERVE * N
    return {
        "value": N * args.steps / wall,
        "ms_per_step": wall * 1000.0 / args.steps,
        "roofline": {
            "bound": "hbm",
            "kernel": f"observe_kernel<{W}>",
            "achieved": nbytes / obs_s / 1e9,
            "peak": PEAK_HBM_BPS / 1e9,
            "unit": "GB/s",
            "frac": nbytes / obs_s / PEAK_HBM_BPS,
            "traffic": None,
            "bytes_per_launch": nbytes,
            "avg_launch_us": obs_s * 1e6,
            "timed_launches": len(obs_events),  # HIP events on one timed step in EVENT_EVERY (event_slots)
        },
        "goal_hits_in_timed_steps": int(cursor.sum().item()) - hits0,
        "resets": int(episodes.sum().item()),
        "device": torch.cuda.get_device_name(0),
    }


def main_costtracer(args) -> int:
    base = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        base = cpu_baseline_costtracer(args)
    res = run_gpu_costtracer(args)
    line = {
        "metric": "agent-steps/sec incl. obs/token build on 1 GPU; % of HBM roofline",
        "value": res["value"],
        "unit": "agent-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16/int32 (integer) + float32 observations",
        "data": "synthetic (seeded i.i.d. maps p=0.2, largest component; distinct starts/goals; goal streams "
                "of free cells; uniform random actions)",
        "config": {
            "workload": "CostTracer environment step: step + reward/goal streams + distance refresh + "
                        "2x11x11 observation + reset",
            "envs": args.envs,
            "agents": args.agents,
            "map": f"{args.map}x{args.map}",
            "task_mode": "costtracer",
            "horizon": args.ct_horizon,
        },
        "roofline": res["roofline"],
        "cpu_baseline": base,
        "goal_hits_in_timed_steps": res["goal_hits_in_timed_steps"],
        "device": res["device"],
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n", 1)[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--envs", type=int, default=1024)
    p.add_argument("--agents", type=int, default=128)
    p.add_argument("--map", type=int, default=64)
    p.add_argument("--seed", type=int, default=20260728)
    p.add_argument("--cpu-envs", type=int, default=2)
    p.add_argument("--cpu-steps", type=int, default=24)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--copy-calibration", action="store_true",
                   help="only run 3 device copies of 256 MiB (PMC byte-counter calibration)")
    p.add_argument("--fetch-probe", action="store_true",
                   help="only run 3 x 1,048,576 isolated 16-byte reads (HBM fetch granularity under FETCH_SIZE)")
    p.add_argument("--graph", action="store_true",
                   help="replay each step from a captured HIP graph (iclr_2027_jointoom_amd/graphs.py)")
    p.add_argument("--workload", choices=("resident", "magat", "c5", "ring", "costtracer", "fresh"),
                   default="resident",
                   help="resident: the north-star MAPF-GPT loop (C2+C3); magat: the C4 MAGAT stateful "
                        "step; c5: the resident loop at C5 (256 envs x 1024 agents, 256x256 warehouses); "
                        "ring: C5 frozen records streamed through the HBM ring into build_tokens; "
                        "costtracer: the CostTracer RL environment step at the C2 shape; fresh: C3 builds with "
                        "every goal fresh (all BFS fields, maze maps by default)")
    p.add_argument("--map-kind", choices=("iid", "maze", "warehouse"), default="iid")
    p.add_argument("--ring-workers", type=int, default=8, help="record producer processes (ring workload)")
    p.add_argument("--ring-slots", type=int, default=4,
                   help="stage slots of the ring (ring workload; 16 unless given)")
    p.add_argument("--ring-compact-only", action="store_true",
                   help="skip the row-format comparison run (ring workload)")
    p.add_argument("--ct-horizon", type=int, default=512, help="episode horizon (costtracer workload)")
    p.add_argument("--policy", choices=("random", "mlp"), default=None,
                   help="resident/c5: pre-staged uniform random actions (the C2 spec) or a random-init token "
                        "MLP in PyTorch choosing them (the C5 spec, its default)")
    p.add_argument("--task-mode", choices=("standard_mapf", "lifelong"), default="standard_mapf",
                   help="resident workload: standard MAPF, or lifelong with deterministic candidate goals")
    args = p.parse_args()
    if args.workload == "ring":
        # 16 stage slots (109 MB of HBM ring, 38 MB of host ring at C5): the
        # producers stay far enough ahead that the ring never runs dry
        for flag, name, value in (("--envs", "envs", 256), ("--agents", "agents", 1024),
                                  ("--map", "map", 256), ("--map-kind", "map_kind", "warehouse"),
                                  ("--steps", "steps", 40), ("--warmup", "warmup", 4),
                                  ("--cpu-steps", "cpu_steps", 3), ("--ring-slots", "ring_slots", 16)):
            if flag not in sys.argv:
                setattr(args, name, value)
    if args.policy is None:
        args.policy = "mlp" if args.workload == "c5" else "random"
    if args.workload == "c5":
        for flag, name, value in (("--envs", "envs", 256), ("--agents", "agents", 1024),
                                  ("--map", "map", 256), ("--map-kind", "map_kind", "warehouse"),
                                  ("--steps", "steps", 50), ("--warmup", "warmup", 3),
                                  ("--cpu-envs", "cpu_envs", 1), ("--cpu-steps", "cpu_steps", 3)):
            if flag not in sys.argv:
                setattr(args, name, value)
    if args.workload == "magat":
        # C4 defaults unless given explicitly
        if "--envs" not in sys.argv:
            args.envs = 512
        if "--agents" not in sys.argv:
            args.agents = 256
        if "--steps" not in sys.argv:
            args.steps = 50
        if "--cpu-steps" not in sys.argv:
            args.cpu_steps = 2000  # ~2 s per worker of the C restatement
    if args.copy_calibration:
        copy_calibration()
        return 0
    if args.fetch_probe:
        fetch_probe()
        return 0
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build's hot path is per-env data parallel with no "
            "cross-GPU exchange, and multi-GPU runs are not part of it. Use --gpus 1.",
            file=sys.stderr,
        )
        return 2
    if args.workload == "magat":
        return main_magat(args)
    if args.workload == "fresh":
        if "--map-kind" not in sys.argv:
            args.map_kind = "maze"
        if "--steps" not in sys.argv:
            args.steps = 10
        if "--warmup" not in sys.argv:
            args.warmup = 2
        return main_fresh(args)
    if args.workload == "ring":
        return main_ring(args)
    if args.workload == "costtracer":
        if "--steps" not in sys.argv:
            args.steps = 100
        if "--cpu-steps" not in sys.argv:
            args.cpu_steps = 40
        return main_costtracer(args)
    base = None
    if not args.no_cpu_baseline:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        base = cpu_baseline_sampled(args, records=False) if args.workload == "c5" else cpu_baseline(args)
    res = run_gpu(args)
    ach = achievable_bandwidth()
    # the build moves about 3 bytes written per 2 read: between the copy and
    # the write-only streams
    ach["build_frac_of_copy"] = res["roofline"]["achieved"] / ach["copy_GBps"]
    ach["build_frac_of_write"] = res["roofline"]["achieved"] / ach["write_GBps"]
    ach["step_frac_of_copy"] = res["step_effective_GBps"] / ach["copy_GBps"]
    res["roofline"]["achievable_copy_GBps"] = ach["copy_GBps"]
    res["roofline"]["frac_of_achievable_copy"] = ach["build_frac_of_copy"]
    line = {
        "metric": "agent-steps/sec incl. obs/token build on 1 GPU; % of HBM roofline",
        "value": res["value"],
        "unit": "agent-steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16/int32 (integer)",
        "data": (
            "synthetic (seeded "
            + {"iid": "i.i.d. maps p=0.2", "maze": "recursive-backtracker mazes",
               "warehouse": "warehouse maps (2x8 shelves, 2-wide aisles)"}[args.map_kind]
            + ", largest component; distinct starts/goals; "
            + ("actions from a random-init token MLP)" if args.policy == "mlp" else "uniform random actions)")
        ),
        "config": {
            "workload": (
                "resident step + MAPF-GPT token build (C5 shape)" if args.workload == "c5"
                else "resident step + MAPF-GPT token build (C2+C3 shape)"
            ),
            "launch": "hip-graph replay" if args.graph else "eager",
            "policy": "random-init token MLP (PyTorch, bf16 256-64-5)" if args.policy == "mlp"
                      else "pre-staged random actions",
            "envs": args.envs,
            "agents": args.agents,
            "map": f"{args.map}x{args.map}",
            "task_mode": args.task_mode,
        },
        "roofline": res["roofline"],
        "cpu_baseline": base,
        "gpu_ms_per_step": res["gpu_ms_per_step"],
        "step_effective_GBps": res["step_effective_GBps"],
        "step_frac_of_peak": res["step_frac_of_peak"],
        "achievable": ach,
        "first_build_ms": res["first_build_ms"],
        "goals_reassigned": res["goals_reassigned"],
        "device": res["device"],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
