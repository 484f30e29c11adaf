"""Build the gfx950 HIP library in-tree.

``python maba-v2-architecture_amd/build_hip.py`` (or ``__graft_entry__.build()``)
compiles every ``csrc/*.hip`` with hipcc for gfx950 only and links
``maba_sparse/_lib/libmaba_hip.so``.  Objects go to ``_build/`` next to this
file.  Every HIP translation unit is built with packed-FP32 instruction
selection disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_DIR = os.path.join(HERE, "maba_sparse", "_lib")
LIB = os.path.join(LIB_DIR, "libmaba_hip.so")

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(REPO, "include"),
]


def _run(cmd):
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that noise.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def compile_objects(sources, obj_dir, extra=()):
    os.makedirs(obj_dir, exist_ok=True)
    objs = []
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        for src in sources:
            obj = os.path.join(obj_dir, os.path.basename(src) + ".o")
            objs.append(obj)
            jobs.append(ex.submit(_run, [HIPCC, *FLAGS, *extra, "-c", src, "-o", obj]))
        for j in jobs:
            j.result()
    return objs


def link(objs, out):
    os.makedirs(os.path.dirname(out), exist_ok=True)
    tmp = out + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, out)


def build_library() -> str:
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = compile_objects(sources, OBJ_DIR)
    link(objs, LIB)
    return LIB


def build_test_probes() -> str:
    src = os.path.join(REPO, "tests", "hip", "mfma_probe.hip")
    out_dir = os.path.join(REPO, "tests", "hip", "_build")
    objs = compile_objects([src], out_dir)
    out = os.path.join(out_dir, "libmfma_probe.so")
    link(objs, out)
    return out


def clean() -> None:
    shutil.rmtree(OBJ_DIR, ignore_errors=True)


if __name__ == "__main__":
    print(build_library())
    print(build_test_probes())
