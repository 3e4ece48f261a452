"""Builds ``akv_amd/libakv_amd.so`` for gfx950 with hipcc (no GPU needed).

Every translation unit is compiled to an object under ``akv_amd/_build/``
in parallel, then linked into one shared library next to this file.  Device
code is compiled with ``-ffp-contract=off`` (the Reposition arithmetic must
round every product and sum separately) and without the packed-fp32
instructions.

Usage: ``python -m akv_amd.build`` or ``akv_amd.build.build()``.
"""

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT_DIR = HERE / "_build"
LIBRARY = HERE / "libakv_amd.so"
ARCH = "gfx950"

HIP_SOURCES = [
    "common.hip", "reposition.hip", "compact.hip", "compact_pages.hip", "decode_meta.hip", "decode_attention.hip",
    "context_attention.hip", "bind_occurrences.hip", "kv_transfer.hip", "gather_slots.hip",
]
CXX_SOURCES = ["event_plan.cpp", "occurrence_window.cpp", "ownership.cpp"]

COMMON_FLAGS = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-Wno-unused-result"]
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc():
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the akv_amd library needs ROCm's hipcc")
    return found


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}):\n{' '.join(cmd)}\n{proc.stdout}")
    return proc.stdout


def build(verbose=False):
    """Compile and link the library; returns its path."""
    hipcc = _hipcc()
    OUT_DIR.mkdir(exist_ok=True)
    jobs = []
    for name in HIP_SOURCES:
        obj = OUT_DIR / (name + ".o")
        jobs.append([hipcc, *COMMON_FLAGS, *HIP_FLAGS, "-c", str(CSRC / name), "-o", str(obj)])
    for name in CXX_SOURCES:
        obj = OUT_DIR / (name + ".o")
        jobs.append([hipcc, *COMMON_FLAGS, "-x", "c++", "-c", str(CSRC / name), "-o", str(obj)])
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(workers) as pool:
        for out in pool.map(_run, jobs):
            if verbose and out.strip():
                print(out, file=sys.stderr)
    objects = [str(OUT_DIR / (n + ".o")) for n in HIP_SOURCES + CXX_SOURCES]
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", str(tmp)])
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
