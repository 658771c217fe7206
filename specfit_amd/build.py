"""Builds the gfx950 HIP library ``lib/libspecfit_amd.so`` in-tree with hipcc.

The library is the C-ABI declared in include/specfit_amd.h; the Python layer
loads it with ctypes.  Usage: ``python -m specfit_amd.build``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(ROOT_DIR, "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libspecfit_amd.so")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
OFFLOAD_ARCH = "gfx950"

SOURCES = ("abi.hip", "router.hip", "dispatch.hip", "swiglu.hip", "combine.hip",
           "attention.hip", "norm.hip", "codec.hip")

HIPCC_FLAGS = (
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # The router's bit-exact contract relies on no implicit contraction; all
    # intended fused multiply-adds are written explicitly.
    "-ffp-contract=off",
    # Never emit packed fp32 arithmetic.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return path


def _run(cmd: list[str]) -> str:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False) -> str:
    """Compile every HIP source into LIB_PATH (always recompiles): one hipcc
    process per source file in parallel, then one link."""
    os.makedirs(LIB_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    objs = [os.path.join(OBJ_DIR, os.path.splitext(s)[0] + ".o") for s in SOURCES]
    cmds = [[cc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-c", os.path.join(CSRC_DIR, s), "-o", o]
            for s, o in zip(SOURCES, objs)]
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(jobs) as pool:
        errs = list(pool.map(_run, cmds))
    tmp = LIB_PATH + ".tmp"
    errs.append(_run([cc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *objs,
                      "-o", tmp]))
    if verbose:
        for err in errs:
            if err.strip():
                print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
