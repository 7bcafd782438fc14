"""Builds libcrosslane.so in-tree with hipcc for gfx950 (no JIT cache).

Every source is compiled to its own object in parallel (each carries its own
gfx950 code object; no relocatable device code is needed), then linked once.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libcrosslane.so")
OBJDIR = os.path.join(PKG, "_build")
SOURCES = ["xl_kernels.hip", "xl_layer.hip", "xl_stream.hip", "xl_stream_iq1.hip", "xl_stream_mix.hip",
           "xl_grouped.hip", "xl_per32.hip", "xl_hc.hip", "xl_exact.hip", "xl_noalloc.hip", "xl_api.cpp"]
HEADERS = ["xl_format.hpp", "xl_rows.hpp", "xl_internal.hpp", "xl_dev.hpp", "xl_iq2.hpp", "xl_stream.hpp", "xl_refexp.hpp", "xl_codebooks.inc",
           "exports.map"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("XL_OFFLOAD_ARCH", "gfx950")
CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC",
    # IEEE-exact arithmetic: no implicit FMA contraction, no fast math.
    "-ffp-contract=off", "-fno-fast-math",
    # Packed-FP32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Keep single-lane atomics as issued: the atomic optimizer rewrites them to
    # broadcast their result at once, which stalls on the return value.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
]
LDFLAGS = [f"--offload-arch={ARCH}", "-shared", "-fPIC", f"-Wl,--version-script={os.path.join(CSRC, 'exports.map')}"]


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(OBJDIR, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc build of {src} failed")
    return obj


def build(verbose: bool = False, jobs: int = 0) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    jobs = jobs or max(1, min(len(SOURCES), os.cpu_count() or 1))
    with ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *LDFLAGS, *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc link of libcrosslane.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
