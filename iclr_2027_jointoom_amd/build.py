"""Build libjointloom.so (the gfx950 C-ABI library) in-tree with hipcc."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
SOURCES = ["jl_sim.hip", "jl_mapfgpt.hip", "jl_energy.hip", "jl_magat.hip", "jl_records.hip",
           "jl_costtracer.hip", "jl_stream.hip"]
OUTPUT = PKG_DIR / "libjointloom.so"

# Packed FP32 VALU forms are disabled for all device code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    return str(candidate) if candidate.exists() else "hipcc"


def build(verbose: bool = False) -> Path:
    """Compile every HIP source into OUTPUT (always recompiles)."""
    tmp = OUTPUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), *[str(CSRC / s) for s in SOURCES]]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stderr}")
    if verbose and proc.stderr:
        print(proc.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
