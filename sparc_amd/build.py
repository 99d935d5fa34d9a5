"""Builds libsparc_hip.so (gfx950) in-tree with hipcc.

``python -m sparc_amd.build`` or ``sparc_amd.build.build()``.  Every call
recompiles.  The objects are compiled in parallel, one process per source
(scan.hip in several parts, one per (transition, I/O dtype) launcher).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libsparc_hip.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
SOURCES = ["scan.hip", "pointwise.hip", "mixer.hip", "norm.hip", "fold.hip"]
# scan.hip compiles as SCAN_PARTS translation units (SPARC_SCAN_PART = 0..11:
# the C ABI, then one per (transition, I/O dtype) launcher), in parallel
SCAN_PARTS = 12
ARCH = os.environ.get("SPARC_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # no packed fp32 VALU instructions (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (ROCm is required to build libsparc_hip.so)")
    return path


def _compile(job: tuple[str, int | None], build_dir: str, extra: list[str]) -> str:
    src, part = job
    stem = os.path.splitext(src)[0] + ("" if part is None else f"_part{part}")
    obj = os.path.join(build_dir, stem + ".o")
    defs = [] if part is None else [f"-DSPARC_SCAN_PART={part}"]
    cmd = [_hipcc(), *HIPCC_FLAGS, *defs, *extra, "-I", INCLUDE, "-I", CSRC, "-c",
           os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def build(verbose: bool = False, extra: list[str] | None = None) -> str:
    extra = list(extra or [])
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    jobs = [(src, part) for src in SOURCES
            for part in (range(SCAN_PARTS) if src == "scan.hip" else [None])]
    # the scan parts are the long ones: start them first
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 4)) as pool:
        objs = list(pool.map(lambda j: _compile(j, build_dir, extra), jobs))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])
