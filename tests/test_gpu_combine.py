"""The fixed-order combine on the device, byte for byte.

The reference's combine check (engine/strata/warm/other_combine_check.cpp:28-48)
sweeps dims 1..4096 and 1..16 picks over random-exponent values with signed
zeros and denormals, shuffled ids, and compares the candidate's bytes with
the original loop (runtime.cpp:183-188: ascending id, fma from +0, then +
shared). Here the same sweep runs through xl_combine_async against the
oracle's combine (pinned to the reference's own other_combine.hpp build by
golden vectors); the device runs round-to-nearest only, so the reference's
other rounding modes do not apply. Then every single-launch kernel's own
combine is checked the same way on the rows it combined (the parity trace's
y), with weights and shared rows that hold signed zeros and denormals.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.test_gpu_grouped import token_routes
from tests.test_gpu_parity import dev, route, step, types_map
from tests.test_gpu_trace import layer_types

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 72641


def values(rng, n):
    """Random sign and mantissa, biased exponent 0..189 (denormals included, no inf/NaN)."""
    bits = (rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32) & np.uint32(0x807FFFFF)) | (
        rng.integers(0, 190, size=n).astype(np.uint32) << np.uint32(23))
    return bits.view(np.float32)


def special_weights(k):
    w = np.array([0.0, -0.0, 1e-40, -3.5, 2.0**20, 0.25, -1e-42, 7.0] * 2, np.float32)[:k]
    return w


@pytest.fixture(scope="module")
def lane():
    ln = xl.Lane(256, 256, 1, 4, types_map(1, 4, 16, 17), max_picks=8)
    yield ln
    ln.close()


def test_device_combine_byte_sweep(orc, lane):
    rng = np.random.default_rng(SEED)
    cases = 0
    for dim in (1, 7, 8, 9, 63, 256, 257, 4096):
        for n in (1, 2, 3, 6, 8, 16):
            step(f"combine sweep dim={dim} picks={n}")
            ids = rng.permutation(n).astype(np.int32)
            w = values(rng, n)
            shared = values(rng, dim)
            rows = values(rng, n * dim).reshape(n, dim)
            rows[:, 0] = np.where(np.arange(n) % 2 == 1, np.float32(-0.0), np.float32(0.0))
            if dim > 1:
                rows[:, 1] = (np.arange(n, dtype=np.uint32) + 1).view(np.float32)   # the smallest denormals
            for sh in (shared, None):
                out = torch.full((dim,), float("nan"), dtype=torch.float32, device="cuda")
                lane.combine_async(dev(ids), dev(w), dev(rows), out, shared=None if sh is None else dev(sh))
                lane.sync()
                want = orc.combine(ids, w, rows, sh)
                assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32)), (dim, n, sh is None)
                cases += 1
    assert cases == 96


def test_device_combine_rejects(lane):
    ids = dev(np.zeros(17, np.int32)); w = dev(np.ones(17, np.float32))
    rows = dev(np.zeros((17, 8), np.float32)); out = torch.zeros(8, dtype=torch.float32, device="cuda")
    with pytest.raises(xl.XLError, match="pick count"):
        lane.combine_async(ids, w, rows, out)


# (XL_LAYER_PATH, dim, ff, E, k, kind, kernel): every single-launch kernel's in-kernel combine
KERNEL_CASES = [
    ("1", 4096, 3072, 12, 6, "iq2", 1),
    ("1", 4096, 3072, 12, 1, "iq2", 1),
    ("1", 4096, 3072, 12, 6, "iq1", 1),
    ("1", 4096, 3072, 12, 6, "mixed", 1),
    ("1", 1024, 512, 8, 8, "mixed", 1),
    ("3", 4096, 3072, 12, 6, "mixed", 3),
    ("3", 1024, 512, 8, 5, "iq1", 3),
]


@pytest.mark.parametrize("path,dim,ff,E,k,kind,kernel", KERNEL_CASES)
def test_kernel_combine_bit_exact(orc, monkeypatch, path, dim, ff, E, k, kind, kernel):
    monkeypatch.setenv("XL_LAYER_PATH", path)
    step(f"in-kernel combine path={path} dim={dim} ff={ff} k={k} {kind}")
    types = layer_types(kind, E)
    ln = xl.Lane(dim, ff, 1, E, types, max_picks=8)
    try:
        ln.generate(SEED)
        rng = np.random.default_rng(dim + k)
        ids, _ = route(rng.standard_normal(E).astype(np.float32), k)
        w = special_weights(k)
        x = rng.standard_normal(dim).astype(np.float32)
        shared = rng.standard_normal(dim).astype(np.float32)
        shared[:4] = [0.0, -0.0, 1e-41, -1e-39]
        out = torch.zeros(dim, dtype=torch.float32, device="cuda")
        y = torch.full((k, dim), float("nan"), dtype=torch.float32, device="cuda")
        ran = ln.layer_trace_async(0, dev(ids), dev(w), dev(x), out, shared=dev(shared), y=y)
        ln.sync()
        assert ran == kernel
        yv = y.cpu().numpy()
        assert np.isfinite(yv).all()
        want = orc.combine(ids, w, yv, shared)
        assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    finally:
        ln.close()


def test_grouped_combine_bit_exact(orc, monkeypatch):
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    dim, ff, E, T, k = 1024, 512, 8, 24, 6
    step(f"grouped combine dim={dim} ff={ff} T={T} k={k}")
    ln = xl.Lane(dim, ff, 1, E, types_map(1, E, 16, 17), max_picks=8, max_tokens=32)
    try:
        ln.generate(SEED)
        rng = np.random.default_rng(11)
        ids, _ = token_routes(rng, T, E, k, None)
        w = np.tile(special_weights(k), (T, 1)).astype(np.float32)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        shared = rng.standard_normal((T, dim)).astype(np.float32)
        shared[:, 0] = -0.0
        out = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        y = torch.full((T * k, dim), float("nan"), dtype=torch.float32, device="cuda")
        ln.grouped_trace_async(0, dev(ids), dev(w), dev(x), out, shared=dev(shared), y=y)
        ln.sync()
        yv = y.cpu().numpy().reshape(T, k, dim)
        got = out.cpu().numpy()
        for t in range(T):
            want = orc.combine(ids[t], w[t], yv[t], shared[t])
            assert np.array_equal(got[t].view(np.uint32), want.view(np.uint32)), t
    finally:
        ln.close()
