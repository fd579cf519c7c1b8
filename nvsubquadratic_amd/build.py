"""Builds ``libnsq_hip.so`` in-tree with hipcc for gfx950.

Each ``csrc/*.hip`` translation unit is compiled to an object in parallel and
the objects are linked into one shared library next to this file.  Flags:

* ``--offload-arch=gfx950`` only (no other targets, no host fallback);
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed-FP32 VALU
  instructions in device code (hipcc's host pass warns that it does not know
  the feature; that warning is harmless and filtered).
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys


HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libnsq_hip.so")

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    p = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(ln for ln in (p.stderr or "").splitlines() if "not a recognized feature" not in ln)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_library(jobs: int | None = None, verbose: bool = True) -> str:
    """Compile every csrc/*.hip and link libnsq_hip.so; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = []
    cmds = []
    for s in srcs:
        o = os.path.join(OBJ_DIR, os.path.basename(s)[:-4] + ".o")
        objs.append(o)
        cmds.append([HIPCC, *FLAGS, "-c", s, "-o", o])
    jobs = jobs or min(len(cmds), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build_library()
