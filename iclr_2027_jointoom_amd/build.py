"""Build the gfx950 libraries in-tree with hipcc.

libjointloom.so is the product: the C ABI of include/jointloom.h.
libjl_bench.so holds the HBM streaming probe that only bench.py (and its
test) loads for the achievable-bandwidth figure; it is not part of the path.
Each source compiles to its own object in parallel, then each library links.
"""
from __future__ import annotations

import os
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
SOURCES = ["jl_sim.hip", "jl_mapfgpt.hip", "jl_energy.hip", "jl_magat.hip", "jl_records.hip",
           "jl_costtracer.hip"]
BENCH_SOURCES = ["bench/jl_stream.hip"]
OUTPUT = PKG_DIR / "libjointloom.so"
BENCH_OUTPUT = PKG_DIR / "libjl_bench.so"

# Packed FP32 VALU forms are disabled for all device code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{CSRC}",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    return str(candidate) if candidate.exists() else "hipcc"


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stderr}")
    return proc.stderr


def _jobs() -> int:
    """Parallel compiles: the CPUs this process may use, at most 16."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link OUTPUT and BENCH_OUTPUT (always
    recompiles)."""
    with tempfile.TemporaryDirectory(prefix="jl_build_") as tmp:
        objs = {src: Path(tmp) / (src.replace("/", "_") + ".o") for src in SOURCES + BENCH_SOURCES}
        cmds = [[hipcc(), *HIPCC_FLAGS, "-c", "-o", str(obj), str(CSRC / src)] for src, obj in objs.items()]
        with ThreadPoolExecutor(max_workers=min(_jobs(), len(cmds))) as pool:
            logs = list(pool.map(_run, cmds))
        for out, srcs in ((OUTPUT, SOURCES), (BENCH_OUTPUT, BENCH_SOURCES)):
            part = out.with_suffix(".so.tmp")
            logs.append(_run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(part),
                              *[str(objs[s]) for s in srcs]]))
            os.replace(part, out)
    if verbose:
        for log in logs:
            if log:
                print(log)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
