"""Build recipe for the in-tree HIP library kraken_amd/libkrk_mi355x.so.

hipcc compiles each source for gfx950 only (no other targets, no CUDA path)
with packed-FP32 instructions disabled, then links one shared library whose
only exported interface is the C ABI in include/krk_mi355x.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkrk_mi355x.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["backend.cpp", "synth.cpp", "gguf.cpp", "gemv.hip", "gemv_digits.hip", "gemv_stream.hip", "dequant.hip", "gemm.hip",
           "gemm_i8.hip", "router.hip", "moe.hip"]

COMMON = ["-O3", "-std=c++17", "-fPIC", "-Wall", "-I", os.path.join(ROOT, "include"),
          "-I", CSRC]
DEVICE = ["--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
          "-packed-fp32-ops", "-munsafe-fp-atomics"]


def _stale(path: str, obj: str) -> bool:
    """The object is older than its source or than any header it may include."""
    if not os.path.exists(obj):
        return True
    deps = [path] + [os.path.join(d, f) for d in (CSRC, os.path.join(ROOT, "include"))
                     for f in os.listdir(d) if f.endswith((".h", ".hpp"))]
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(d) > t for d in deps)


def _compile(src: str, force: bool = True) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    if not force and not _stale(path, obj):
        return obj
    if src.endswith(".hip") or src == "backend.cpp":
        cmd = [HIPCC, *COMMON, *DEVICE, "-x", "hip", "-c", path, "-o", obj]
    else:
        cmd = [HIPCC, *COMMON, "-x", "c++", "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    # hipcc's host pass does not know the device-only feature; that line is noise
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs: int | None = None, force: bool = True) -> str:
    """Compile every source (force=False: only those whose object is stale)
    and link the library."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, len(SOURCES))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--changed" not in sys.argv))
