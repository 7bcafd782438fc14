"""GPU parity of the per32 mode (the reference's production HIP lane
arithmetic, engine/strata/warm/hip_experts.hip) against the oracle's per32
restatement, through the C ABI.

Bars: per-32 quants and scales bit-exact; matvec rows bit-exact (same integer
dots, same float rounding order: scale * int, fma into the lane, xor butterfly);
the layer's per-pick outputs within max relative error 1e-3 of the oracle chain
(the SwiGLU's exp differs by ulps between host and device, which can move a
hidden quant by one); combine bit-exact against the oracle's fixed-order combine
of the device's own per-pick rows; runs bit-identical.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import crosslane_amd as xl
from oracle.oracle import BLOCK_BYTES
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu
TOL = 1e-3

torch = pytest.importorskip("torch")


def step(msg):
    print(f"[gpu-step] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def types_map(L, E, gu, dn):
    t = np.zeros((L, E, 3), np.int32)
    t[..., 0] = gu; t[..., 1] = gu; t[..., 2] = dn
    return t


@pytest.fixture(scope="module")
def probe():
    lane = xl.Lane(4096, 4096, 1, 1, types_map(1, 1, 16, 16), max_picks=1)
    yield lane
    lane.close()


def quant_cases(rng):
    ties = np.tile(np.arange(32, dtype=np.float32) - 15.5, 1)
    ties[0] = 127.0                      # d = 1: every other value a half-way case
    cases = [np.zeros(64, np.float32), ties]
    for scale in (1e-30, 1e-3, 1.0, 1e4):
        cases.append((rng.standard_normal(4096) * scale).astype(np.float32))
    mixed = rng.standard_normal(3072).astype(np.float32)
    mixed[32:64] = 0.0                   # an all-zero block amid others
    cases.append(mixed)
    return cases


def test_quant32_bit_exact(probe, orc, rng):
    for x in quant_cases(rng):
        step(f"quant32 n={x.size}")
        q = torch.zeros(x.size, dtype=torch.int8, device="cuda")
        d = torch.zeros(x.size // 32, dtype=torch.float32, device="cuda")
        probe.quantize_per32_async(dev(x), 1, x.size, q, d)
        probe.sync()
        wq, wd = orc.quant32(x)
        assert np.array_equal(q.cpu().numpy(), wq)
        assert np.array_equal(d.cpu().numpy().view(np.uint32), wd.view(np.uint32))


def test_quant32_rows(probe, orc, rng):
    x = rng.standard_normal((6, 3072)).astype(np.float32)
    step("quant32 rows=6 k=3072")
    q = torch.zeros(x.size, dtype=torch.int8, device="cuda")
    d = torch.zeros(x.size // 32, dtype=torch.float32, device="cuda")
    probe.quantize_per32_async(dev(x), 6, 3072, q, d)
    probe.sync()
    wq, wd = orc.quant32(x.reshape(-1))   # blocks of 32 never straddle rows
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(d.cpu().numpy(), wd)


@pytest.mark.parametrize("t", [16, 17, 29])
@pytest.mark.parametrize("n,k", [(64, 256), (40, 768), (64, 1024), (24, 2048), (256, 3072), (256, 4096)])
def test_matvec32_bit_exact(probe, orc, t, n, k):
    step(f"matvec32 type={t} n={n} k={k}")
    aos = orc.gen_matrix(t, 777 + k, 0, t, 1, n, k)
    x = np.random.default_rng(n * k + t).standard_normal(k).astype(np.float32)
    q, d = orc.quant32(x)
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    probe.matvec_per32_async(t, dev(xl.repack(t, n, k, aos)), n, k, dev(q), dev(d), y)
    probe.sync()
    want = orc.matvec32(t, aos, n, k, q, d)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_matvec32_rows_against_row32(probe, orc):
    """Every row also equals the single-row restatement (orc_row32)."""
    t, n, k = 29, 16, 4096
    aos = orc.gen_matrix(t, 31, 0, 0, 2, n, k)
    x = np.random.default_rng(3).standard_normal(k).astype(np.float32) * 7.0
    q, d = orc.quant32(x)
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    step("matvec32 vs row32")
    probe.matvec_per32_async(t, dev(xl.repack(t, n, k, aos)), n, k, dev(q), dev(d), y)
    probe.sync()
    rb = (k // 256) * BLOCK_BYTES[t]
    want = np.array([orc.row32(t, aos[r * rb:(r + 1) * rb], k, q, d) for r in range(n)], np.float32)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


# ---- layer ---------------------------------------------------------------------------
SEED = 0x9E32
LAYER_TYPES = {0: (16, 16, 17), 1: (29, 29, 29)}


@pytest.fixture(scope="module")
def lane32():
    step("per32 lane: 4096x3072, 2 layers x 64 experts (IQ2_XXS/IQ2_XS, IQ1_M)")
    t = np.zeros((2, 64, 3), np.int32)
    for layer, ty in LAYER_TYPES.items():
        t[layer, :] = ty
    lane = xl.Lane(4096, 3072, 2, 64, t, max_picks=8)
    lane.generate(seed=SEED)
    yield lane
    lane.close()


@pytest.mark.parametrize("layer", [0, 1])
def test_layer_per32_vs_oracle(lane32, orc, layer):
    rng = np.random.default_rng(40 + layer)
    ids = rng.choice(64, 6, replace=False).astype(np.int32)
    w = rng.random(6).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    shared = rng.standard_normal(4096).astype(np.float32)
    step(f"per32 layer={layer} ids={ids.tolist()}")
    y, out = lane32.layer_forward_per32(layer, ids, x, w, shared)
    ty = LAYER_TYPES[layer]
    want = np.stack([orc.expert32(ty, *orc.gen_expert(ty, SEED, layer, int(e), 4096, 3072), 4096, 3072, x)
                     for e in ids])
    for i in range(6):
        assert max_rel(y[i], want[i]) < TOL, f"pick {i}"
    assert np.array_equal(out.view(np.uint32), orc.combine(ids, w, y, shared).view(np.uint32))


def test_layer_per32_deterministic_async(lane32):
    rng = np.random.default_rng(50)
    ids = rng.choice(64, 6, replace=False).astype(np.int32)
    w = rng.random(6).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    step("per32 layer determinism + async")
    y0, out0 = lane32.layer_forward_per32(0, ids, x, w)
    for _ in range(2):
        y1, out1 = lane32.layer_forward_per32(0, ids, x, w)
        assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
        assert np.array_equal(out0.view(np.uint32), out1.view(np.uint32))
    yd = torch.zeros((6, 4096), dtype=torch.float32, device="cuda")
    od = torch.zeros(4096, dtype=torch.float32, device="cuda")
    lane32.layer_forward_per32_async(0, dev(ids), dev(x), yd, w=dev(w), out=od)
    lane32.sync()
    assert np.array_equal(yd.cpu().numpy().view(np.uint32), y0.view(np.uint32))
    assert np.array_equal(od.cpu().numpy().view(np.uint32), out0.view(np.uint32))
    y_only, none = lane32.layer_forward_per32(0, ids, x)
    assert none is None and np.array_equal(y_only.view(np.uint32), y0.view(np.uint32))


def test_layer_per32_rejects_bad_input(lane32):
    x = np.zeros(4096, np.float32)
    with pytest.raises(xl.XLError):
        lane32.layer_forward_per32(0, [3, 3], x, [0.5, 0.5])
    with pytest.raises(xl.XLError):
        lane32.layer_forward_per32(0, [64], x)
    bad = torch.tensor([1, 99], dtype=torch.int32, device="cuda")
    yd = torch.zeros((2, 4096), dtype=torch.float32, device="cuda")
    lane32.layer_forward_per32_async(0, bad, dev(x), yd)
    with pytest.raises(xl.XLError):
        lane32.sync()
    with pytest.raises(xl.XLError, match="poisoned"):
        lane32.layer_forward_per32(0, [1], x)
