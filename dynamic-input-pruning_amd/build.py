"""Build libdip_hip.so (the gfx950 DIP decode kernels + C ABI) in-tree.

    python dynamic-input-pruning_amd/build.py

Each csrc/*.hip file is compiled to an object under _build/ (in parallel),
then linked into libdip_hip.so next to this file.  The library is what the
Python modules in this directory load; it is rebuilt every time this runs.
csrc/probe/*.hip (the bench's read-ceiling probes, no part of the decode
path) is linked into a library of its own, libdip_probe.so.  The decode
sources are built a second time with DIP_WG_STAMPS into
libdip_hip_timeline.so, whose decode kernels record per-workgroup timeline
stamps (dip_timeline_read; `bench.py --timeline`).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB = HERE / "libdip_hip.so"
PROBE_LIB = HERE / "libdip_probe.so"
# the same sources with per-workgroup timeline stamps (dip_timeline_read)
TIMELINE_LIB = HERE / "libdip_hip_timeline.so"
ARCH = os.environ.get("DIP_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 math is off for every kernel in this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    err = "\n".join(l for l in proc.stderr.splitlines()
                    if "packed-fp32-ops" not in l and l.strip())
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    return err


def _link(objs, lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
          "-lpthread"])
    os.replace(tmp, lib)


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip and link libdip_hip.so (and csrc/probe/*.hip
    into libdip_probe.so); returns the decode library's path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    probes = sorted((CSRC / "probe").glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(job) -> Path:
        src, timeline = job
        tag = "tl_" if timeline else ""
        obj = BUILD / (tag + src.parent.name + "_" + src.stem + ".o")
        cmd = [HIPCC, *COMMON, *(["-DDIP_WG_STAMPS"] if timeline else []), "-c", str(src), "-o",
               str(obj)]
        msg = _run(cmd)
        if verbose and msg:
            print(msg, file=sys.stderr)
        return obj

    jobs_list = [(p, False) for p in sources + probes] + [(p, True) for p in sources]
    jobs = min(len(jobs_list), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(compile_one, jobs_list))
    n, m = len(sources), len(sources) + len(probes)
    _link(objs[:n], LIB)
    if probes:
        _link(objs[n:m], PROBE_LIB)
    _link(objs[m:], TIMELINE_LIB)
    if verbose:
        print(f"built {LIB}" + (f", {PROBE_LIB}" if probes else "") + f" and {TIMELINE_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
