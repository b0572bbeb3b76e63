"""Build recipe for the in-tree HIP library kraken_amd/libkrk_mi355x.so.

hipcc compiles each source for gfx950 only (no other targets, no CUDA path)
with packed-FP32 instructions disabled, then links one shared library whose
only exported interface is the C ABI in include/krk_mi355x.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
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


def check_dma_waits(asm_text: str, kernel_prefix: str = "_ZN3krk15moe_gemm_kernel"):
    """The grouped expert GEMM publishes each block's activation DMA
    (global_load_lds) with `s_waitcnt vmcnt(N)` followed by a barrier,
    counting on N vector loads (the next block's weights) having been issued
    after the DMA: vector memory completes in order, so at most N
    outstanding then means the DMA has landed.  In every such kernel of the
    emitted gfx950 assembly, each vmcnt(N) right before an s_barrier must
    follow at least N vector loads issued after the last DMA, in program
    order.  Returns (sites checked, [(kernel, line, loads after the DMA, N)]
    of violations)."""
    bad, sites = [], 0
    lines = asm_text.splitlines()
    i = 0
    while i < len(lines):
        if lines[i].startswith(kernel_prefix) and ":" in lines[i]:
            name = lines[i].split(":")[0]
            since = None
            j = i + 1
            while j < len(lines) and "s_endpgm" not in lines[j]:
                t = lines[j].strip()
                if t.startswith("global_load_lds"):
                    since = 0
                elif re.match(r"(global|buffer|flat)_load", t) and since is not None:
                    since += 1
                m = re.match(r"s_waitcnt\s+vmcnt\((\d+)\)", t)
                if m and since is not None and any(x.strip().startswith("s_barrier") for x in lines[j + 1:j + 5]):
                    sites += 1
                    if since < int(m.group(1)):
                        bad.append((name, j + 1, since, int(m.group(1))))
                j += 1
            i = j
        i += 1
    return sites, bad


def _check_gemm_asm() -> None:
    """Emit gemm.hip's device assembly and run check_dma_waits on it."""
    out = os.path.join(BUILD, "gemm.s")
    cmd = [HIPCC, *COMMON, *DEVICE, "-x", "hip", "-S", "--cuda-device-only", os.path.join(CSRC, "gemm.hip"),
           "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"assembly of gemm.hip failed\n{r.stderr}")
    sites, bad = check_dma_waits(open(out).read())
    if sites == 0 or bad:
        raise RuntimeError(f"gemm.hip: DMA publish waits not covered by later loads ({sites} sites): {bad[:4]}")


def build(jobs: int | None = None, force: bool = True) -> str:
    """Compile every source (force=False: only those whose object is stale)
    and link the library."""
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(8, len(SOURCES))
    with cf.ThreadPoolExecutor(jobs) as ex:
        asm_check = ex.submit(_check_gemm_asm) if force or _stale(os.path.join(CSRC, "gemm.hip"),
                                                                   os.path.join(BUILD, "gemm.s")) else None
        objs = list(ex.map(lambda s: _compile(s, force), SOURCES))
        if asm_check is not None:
            asm_check.result()
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(force="--changed" not in sys.argv))
