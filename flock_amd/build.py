"""Build libflock_attn.so in-tree with hipcc for gfx950.

    python -m flock_amd.build

The library is written next to this file (flock_amd/libflock_attn.so) so it
travels with the source tree; nothing is installed into site-packages.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libflock_attn.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",  # rounding points are explicit (fmaf where wanted)
    # Keep hipcc from forming packed-f32 instructions (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libflock_attn.so)")


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every HIP source into flock_amd/libflock_attn.so; returns its path.

    Each source is compiled to an object of its own (in parallel, at most
    `jobs` at a time: default the CPU count, capped at 16), then the objects
    are linked. Objects go to a temporary folder next to the library and are
    removed afterwards."""
    srcs = sources()
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    objs = [os.path.join(objdir, os.path.basename(s) + ".o") for s in srcs]
    jobs = jobs or min(16, os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, [hipcc(), *HIPCC_FLAGS, "-c", "-o", o, s], verbose)
                  for s, o in zip(srcs, objs)]:
            f.result()
    tmp = LIB + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    shutil.rmtree(objdir, ignore_errors=True)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
