"""Build the gfx950 HIP library ``mamba3_rocm/libmamba3_rocm.so`` in-tree.

Plain ``hipcc``: every ``csrc/*.hip`` file is compiled for gfx950 in parallel
and linked into one shared library whose only interface is the C ABI of
``include/mamba3_scan.h``.  Packed-fp32 instructions are disabled in device
code (``-Xclang -target-feature -Xclang -packed-fp32-ops``).

Usage: python sigma-0_amd/build.py [--verbose]
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "mamba3_rocm")
LIB_NAME = "libmamba3_rocm.so"
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
]
# The chunk states come from two instantiations of each chunked kernel: the state-only
# pass (the recomputing backward, the sequence split) and the full pass that saves them
# (the training forward).  HIP's default contraction (fast) lets the backend fuse a
# multiply into a later add across statements, so the same source could round
# differently in the two (a last-bit difference in a rope'd key or a key weight that
# the bf16 operand rounding then occasionally turns into a different state element).
# Contraction within an expression only (on) makes every instantiation compute the
# same operations; it leaves these kernels' instruction counts unchanged to within
# 0.3%.
FILE_CFLAGS = {
    "m3_scan_chunked.hip": ["-ffp-contract=on"],
    "m3_scan_chunked_f32.hip": ["-ffp-contract=on"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the Mamba3 HIP library needs ROCm's hipcc")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{errs}")
    if verbose and errs.strip():
        print(errs)


def build(verbose: bool = False) -> str:
    """Compile and link; returns the path of the shared library."""
    cc = hipcc()
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    srcs = sorted(f for f in os.listdir(CSRC) if f.endswith(".hip"))
    objs = [os.path.join(build_dir, s[:-4] + ".o") for s in srcs]
    t0 = time.time()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        futs = [ex.submit(_run, [cc, *CFLAGS, *FILE_CFLAGS.get(s, []), "-c", os.path.join(CSRC, s), "-o", o], verbose)
                for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    lib = os.path.join(OUT_DIR, LIB_NAME)
    tmp = lib + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib} in {time.time() - t0:.1f}s", flush=True)
    return lib


if __name__ == "__main__":
    build(verbose="--verbose" in sys.argv or "-v" in sys.argv)
