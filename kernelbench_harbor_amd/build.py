"""Builds the HIP kernels of this package into one C-ABI shared library for gfx950.

`build()` compiles every ``csrc/*.hip`` with hipcc (``--offload-arch=gfx950``) into objects
under ``_build/`` and links ``kernelbench_harbor_amd/lib/libkbh_qgemm.so``. It always
recompiles (it is the "does it build" check); ``python -m kernelbench_harbor_amd.build``
does the same from the command line.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
OBJ_DIR = os.path.join(REPO_DIR, "_build", "obj")
LIB_NAME = "libkbh_qgemm.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed fp32 VALU ops stay off: hipcc must not emit v_pk_{add,mul,fma}_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC_DIR, f) for f in os.listdir(CSRC_DIR) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, "-I", INCLUDE_DIR, "-I", CSRC_DIR, "-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    errs = [ln for ln in res.stderr.splitlines()
            if ln.strip() and "packed-fp32-ops" not in ln and "recognized feature" not in ln]
    if errs:
        print(f"[kbh build] {os.path.basename(src)}:\n" + "\n".join(errs[:40]), file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    """Compiles all kernels and links the shared library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    workers = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[kbh build] {len(srcs)} sources -> {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
