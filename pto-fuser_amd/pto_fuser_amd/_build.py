"""Build libptofuser_hip.so in-tree with hipcc for gfx950.

The library is compiled from ``pto-fuser_amd/csrc/*.hip`` into
``pto-fuser_amd/pto_fuser_amd/lib/libptofuser_hip.so``; it travels with the source tree, so a
GPU box loads the file built here.  ``build()`` always recompiles (it is the "does it build"
check); ``ensure_built()`` compiles only when no library exists yet.

Every build embeds :func:`source_hash` (the sources, headers and compiler flags it was made
from) as ``pf_source_hash()``; the loader compares it with the tree's current hash and refuses a
library built from other sources, so an edit without a rebuild never ships a stale library.
"""
from __future__ import annotations

import glob
import hashlib
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from typing import List, Optional

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)                       # pto-fuser_amd/
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(os.path.dirname(ROOT), "include")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_NAME = "libptofuser_hip.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)
ARCH = os.environ.get("PF_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops is disabled: the compiler must not form v_pk_{add,mul,fma}_f32 on its own.
# The iterative-ILP machine scheduler issues the LDS operand reads of the scan's MFMA chains
# several instructions ahead (the default strategy serialises every MFMA behind its own read,
# which leaves a one-wave-per-SIMD kernel latency-bound).
HIPCC_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               "-mllvm", "-amdgpu-sched-strategy=iterative-ilp"]
OBJ_DIR = os.path.join(ROOT, "_build")


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def sources() -> List[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


def headers() -> List[str]:
    return sorted(glob.glob(os.path.join(CSRC, "*.h")) + glob.glob(os.path.join(INCLUDE, "*.h")))


def source_hash() -> str:
    """16 hex digits of SHA-256 over every source and header (name and content) and the hipcc
    flags: what the library's ``pf_source_hash()`` must return for it to be current."""
    h = hashlib.sha256()
    for path in sources() + headers():
        h.update(os.path.basename(path).encode() + b"\0")
        with open(path, "rb") as f:
            h.update(f.read())
        h.update(b"\0")
    h.update(" ".join(HIPCC_FLAGS).encode())
    return h.hexdigest()[:16]


def _run(cmd: List[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"libptofuser_hip build failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = False, out: Optional[str] = None) -> str:
    """Compile every HIP source to an object (one hipcc per translation unit, in parallel), then
    link the shared library; raises RuntimeError with the compiler output on failure.  Returns
    the library path."""
    out = out or LIB_PATH
    os.makedirs(os.path.dirname(out), exist_ok=True)
    obj_dir = os.path.join(OBJ_DIR, str(os.getpid()))
    os.makedirs(obj_dir, exist_ok=True)
    hipcc = _hipcc()
    srcs = sources()
    objs = [os.path.join(obj_dir, os.path.splitext(os.path.basename(s))[0] + ".o") for s in srcs]
    jobs = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", "8"))))
    tag = f'-DPF_SOURCE_HASH="{source_hash()}"'
    try:
        with ThreadPoolExecutor(jobs) as pool:
            list(pool.map(lambda so: _run([hipcc, *HIPCC_FLAGS, tag, "-I", INCLUDE, "-c", so[0],
                                           "-o", so[1]], verbose), zip(srcs, objs)))
        tmp = out + f".tmp{os.getpid()}"
        _run([hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp], verbose)
        os.replace(tmp, out)
    finally:
        shutil.rmtree(obj_dir, ignore_errors=True)
    return out


PROBE_SRC = os.path.join(CSRC, "probe", "pf_memfloor.hip")
PROBE_PATH = os.path.join(LIB_DIR, "pf_memfloor")


def build_probe(verbose: bool = False) -> str:
    """Compile the memory-floor probe (``csrc/probe/pf_memfloor.hip``: the scan kernels' load and
    store traffic with no compute, a measurement tool outside the library) into
    ``lib/pf_memfloor``; returns its path."""
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = PROBE_PATH + f".tmp{os.getpid()}"
    _run([_hipcc(), *[f for f in HIPCC_FLAGS if f != "-fPIC"], PROBE_SRC, "-o", tmp], verbose)
    os.replace(tmp, PROBE_PATH)
    return PROBE_PATH


def ensure_built(verbose: bool = False) -> str:
    """Return the library path, compiling only when no library has been built yet (the GPU box
    runs the library built in this tree; it never rebuilds a present one)."""
    if not os.path.exists(LIB_PATH):
        return build(verbose=verbose)
    return LIB_PATH
