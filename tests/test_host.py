"""CPU: the C-ABI library loads and exports every symbol include/crosslane.h
declares; host-side logic (repack/restore, generator, argument and version
checks) runs without a GPU. No compute call is made here."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np
import pytest

import crosslane_amd as xl
from crosslane_amd import lane as L
from tests.conftest import ROOT


def header_functions():
    text = open(os.path.join(ROOT, "include", "crosslane.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xl_[a-z0-9_]+)\s*\(", text)))


def test_exports_every_declared_symbol():
    lib = C.CDLL(L.LIB_PATH)
    names = header_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(L._SIGNATURES), set(names) ^ set(L._SIGNATURES)


def test_abi_version():
    assert xl.lib().xl_abi_version() == L.ABI_VERSION == 3


def test_open_rejects_version_and_size_before_device():
    cfg = L._Config(C.sizeof(L._Config), 0, 4096, 3072, 1, 384, 8, 0, 0.0)
    ctx, err = C.c_void_p(), L._Err()
    v = L.ABI_VERSION
    assert xl.lib().xl_open(v + 1, C.byref(cfg), C.byref(ctx), C.byref(err)) == 5
    assert b"version" in err.message and not ctx.value
    cfg.struct_bytes = 32   # the version-1 layout (no swiglu_limit)
    assert xl.lib().xl_open(v, C.byref(cfg), C.byref(ctx), C.byref(err)) == 5
    cfg.struct_bytes = C.sizeof(L._Config)
    cfg.dim = 1000
    assert xl.lib().xl_open(v, C.byref(cfg), C.byref(ctx), C.byref(err)) == 1
    assert b"dim" in err.message
    cfg.dim, cfg.max_picks = 4096, 17
    assert xl.lib().xl_open(v, C.byref(cfg), C.byref(ctx), C.byref(err)) == 1
    cfg.max_picks, cfg.swiglu_limit = 8, float("inf")
    assert xl.lib().xl_open(v, C.byref(cfg), C.byref(ctx), C.byref(err)) == 1
    assert b"swiglu_limit" in err.message


@pytest.mark.parametrize("t", [16, 17, 29])
@pytest.mark.parametrize("nk", [(256, 4096), (4096, 3072), (8, 256), (3, 768)])
def test_repack_restore_lossless(orc, t, nk):
    n, k = nk
    aos = orc.gen_matrix(t, 77, 1, 2, 0, n, k)
    planar = xl.repack(t, n, k, aos)
    if (n * k // 256) % 128 == 0:
        assert planar.size == aos.size          # no padding at the benchmark shapes
    assert np.array_equal(xl.restore(t, n, k, planar), aos)


def test_repack_is_a_bit_permutation():
    # The repack moves and re-encodes fields but only permutes bits: every
    # single set bit of a block lands on exactly one planar bit, and back.
    for t in (16, 17, 29):
        bb = L.BLOCK_BYTES[t]
        seen = set()
        for bit in range(8 * bb):
            aos = np.zeros(4 * bb, np.uint8)
            aos[bb + bit // 8] = 1 << (bit % 8)                # block 1 of 4
            planar = xl.repack(t, 1, 1024, aos)
            ones = np.flatnonzero(np.unpackbits(planar))
            assert ones.size == 1
            seen.add(int(ones[0]))
            assert np.array_equal(xl.restore(t, 1, 1024, planar), aos)
        assert len(seen) == 8 * bb


@pytest.mark.parametrize("t", [16, 17, 29])
def test_host_generator_matches_oracle(orc, t):
    for (layer, expert, role) in ((0, 0, 0), (39, 383, 2), (7, 123, 1)):
        a = xl.generate_host(t, 0xC0FFEE, layer, expert, role, 32, 1024)
        b = orc.gen_matrix(t, 0xC0FFEE, layer, expert, role, 32, 1024)
        assert np.array_equal(a, b)


def test_planar_bytes():
    assert xl.planar_bytes(16, 3072, 4096) == 3072 * 16 * 66
    assert xl.planar_bytes(17, 4096, 3072) == 4096 * 12 * 74
    assert xl.planar_bytes(29, 3072, 4096) == 3072 * 16 * 56
    assert xl.planar_bytes(15, 3072, 4096) == 0
