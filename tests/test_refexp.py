"""The exact path's expf (crosslane_amd/csrc/xl_refexp.hpp) against this host's
C library expf, the function the reference's SwiGLU calls (q8k_core.hpp:94)
and the oracle links. CPU only: a small driver is compiled with g++ and
compares every 61st float bit pattern plus the range boundaries bit for bit
(the whole range (-130, 100) was compared once when the header was written:
no mismatch)."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

DRIVER = r"""
#include <cmath>
#include <cstdio>
#include <cstring>
#include "xl_refexp.hpp"
int main() {
    unsigned long long n = 0, bad = 0;
    auto one = [&](float x) {
        const float a = expf(x), b = xl::ref_expf(x);
        ++n;
        if (std::memcmp(&a, &b, 4)) { if (bad < 5) std::printf("x=%a libm=%a ref=%a\n", x, a, b); ++bad; }
    };
    for (unsigned long long u = 0; u <= 0xffffffffull; u += 61) {
        unsigned b = unsigned(u); float x; std::memcpy(&x, &b, 4);
        if (x > -130.0f && x < 100.0f) one(x);
    }
    const float edges[] = {0x1.62e42ep6f, 0x1.62e430p6f, -0x1.9fe368p6f, -0x1.9fe36ap6f, -0x1.9fe366p6f,
                           -87.0f, -0x1.5d589ep6f, 0.0f, -0.0f, 1e-30f, -1e-30f, 88.0f};
    for (float x : edges) one(x);
    std::printf("n=%llu bad=%llu\n", n, bad);
    return bad != 0;
}
"""


def test_ref_expf_matches_host_libm(tmp_path):
    if shutil.which("g++") is None:
        pytest.skip("g++ absent")
    src = tmp_path / "refexp.cpp"
    src.write_text(DRIVER)
    exe = tmp_path / "refexp"
    r = subprocess.run(["g++", "-O2", "-std=c++20", "-ffp-contract=off",
                        f"-I{os.path.join(ROOT, 'crosslane_amd', 'csrc')}", str(src), "-o", str(exe), "-lm"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
