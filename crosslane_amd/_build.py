"""Builds libcrosslane.so in-tree with hipcc for gfx950 (no JIT cache)."""
from __future__ import annotations

import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libcrosslane.so")
SOURCES = ["xl_kernels.hip", "xl_layer.hip", "xl_stream.hip", "xl_grouped.hip", "xl_per32.hip", "xl_hc.hip", "xl_api.cpp"]
HEADERS = ["xl_format.hpp", "xl_rows.hpp", "xl_internal.hpp", "xl_dev.hpp", "xl_codebooks.inc", "exports.map"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("XL_OFFLOAD_ARCH", "gfx950")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-shared",
    # IEEE-exact arithmetic: no implicit FMA contraction, no fast math.
    "-ffp-contract=off", "-fno-fast-math",
    # Packed-FP32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Keep single-lane atomics as issued: the atomic optimizer rewrites them to
    # broadcast their result at once, which stalls on the return value.
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    f"-Wl,--version-script={os.path.join(CSRC, 'exports.map')}",
]


def build(verbose: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    tmp = LIB + ".tmp"
    cmd = [HIPCC, *FLAGS, *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc build of libcrosslane.so failed")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
