"""GPU parity of the steps around the routed experts (hip_backend.cpp:664-666,
777): the shared-expert FFN in the per32 arithmetic over the dense formats
(Q8_0, Q4_K, Q5_K, Q6_K) and the hyper-connection post, through the C ABI.

Bars: dense per32 rows bit-exact against the oracle (itself bit-exact against
the reference's core.hpp lane<> build); the shared FFN within max-rel 1e-3 of
the oracle chain (the SwiGLU's exp differs by ulps between host and device);
hc_post bit-exact (products and sums in the reference's order, one rounding
each); the composition shared FFN -> routed layer (shared row added last) ->
hc_post within 1e-3 of the oracle composition.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.dense import dense_matrix

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
    lane = xl.Lane(4096, 3072, 1, 1, types_map(1, 1, 16, 17), max_picks=1)
    yield lane
    lane.close()


@pytest.mark.parametrize("t", [8, 12, 13, 14])
@pytest.mark.parametrize("n,k", [(64, 256), (40, 1024), (96, 3072), (256, 4096)])
def test_matvec32_dense_bit_exact(probe, orc, t, n, k):
    step(f"dense matvec32 type={t} n={n} k={k}")
    w = dense_matrix(t, n, k, seed=n + k)
    x = (np.random.default_rng(n * k + t).standard_normal(k) * 2.0).astype(np.float32)
    q, d = orc.quant32(x)
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    probe.matvec_per32_async(t, dev(w), n, k, dev(q), dev(d), y)
    probe.sync()
    want = orc.matvec32(t, w, n, k, q, d)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


def shared_mats(types, dim, ff, seed):
    return (dense_matrix(types[0], ff, dim, seed), dense_matrix(types[1], ff, dim, seed + 1),
            dense_matrix(types[2], dim, ff, seed + 2))


@pytest.mark.parametrize("types,ff,T,lim", [((13, 13, 14), 3072, 1, 0.0), ((12, 12, 8), 2048, 3, 0.0),
                                            ((14, 14, 13), 1024, 2, 7.0), ((8, 8, 12), 3072, 1, 7.0)])
def test_shared_forward_vs_oracle(orc, types, ff, T, lim):
    dim = 4096
    step(f"shared FFN types={types} ff={ff} T={T} lim={lim}")
    lane = xl.Lane(dim, 3072, 1, 1, types_map(1, 1, 16, 17), max_picks=1, swiglu_limit=lim)
    try:
        g, u, dn = shared_mats(types, dim, ff, seed=ff + T)
        x = (np.random.default_rng(ff + 7 * T).standard_normal((T, dim)) * 2.0).astype(np.float32)
        work = torch.empty(xl.shared_work_bytes(dim, ff, T), dtype=torch.uint8, device="cuda")
        out = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        lane.shared_forward_async(types, dev(g), dev(u), dev(dn), ff, dev(x), out, work)
        lane.sync()
        got = out.cpu().numpy()
        for t in range(T):
            want = orc.expert32(types, g, u, dn, dim, ff, x[t], limit=lim)
            assert max_rel(got[t], want) < TOL, (t, max_rel(got[t], want))
        again = torch.zeros_like(out)
        lane.shared_forward_async(types, dev(g), dev(u), dev(dn), ff, dev(x), again, work)
        lane.sync()
        assert torch.equal(out, again)
    finally:
        lane.close()


def test_shared_forward_rejects(probe):
    dim, ff = 4096, 1024
    g, u, dn = shared_mats((12, 12, 12), dim, ff, seed=1)
    x = torch.zeros((1, dim), dtype=torch.float32, device="cuda")
    out = torch.zeros_like(x)
    small = torch.empty(xl.shared_work_bytes(dim, ff, 1) - 256, dtype=torch.uint8, device="cuda")
    with pytest.raises(xl.XLError, match="workspace"):
        probe.shared_forward_async((12, 12, 12), dev(g), dev(u), dev(dn), ff, x, out, small)
    work = torch.empty(xl.shared_work_bytes(dim, ff, 1), dtype=torch.uint8, device="cuda")
    with pytest.raises(xl.XLError, match="block type"):
        probe.shared_forward_async((10, 12, 12), dev(g), dev(u), dev(dn), ff, x, out, work)
    assert xl.shared_work_bytes(dim, 1000, 1) == 0


@pytest.mark.parametrize("T,H,D", [(3, 4, 4096), (1, 1, 300), (2, 2, 1000), (5, 3, 64)])
def test_hc_post_bit_exact(probe, orc, T, H, D):
    step(f"hc_post T={T} H={H} D={D}")
    rng = np.random.default_rng(T * 100 + H * 10 + D)
    y = rng.standard_normal((T, D)).astype(np.float32)
    res = rng.standard_normal((T, H, D)).astype(np.float32)
    post = (rng.random((T, 8)) * 2).astype(np.float32)
    comb = rng.random((T, 64)).astype(np.float32)
    want = orc.hc_post(y, res, post, comb, D, H, T)
    out = torch.zeros((T, H, D), dtype=torch.float32, device="cuda")
    dres = dev(res)
    probe.hc_post_async(dev(y), dres, dev(post), dev(comb), out)
    probe.sync()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    probe.hc_post_async(dev(y), dres, dev(post), dev(comb), dres)   # in place (hc_post_inplace)
    probe.sync()
    assert np.array_equal(dres.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("T,H,D", [(1, 1, 4096), (2, 4, 5120), (3, 3, 1500), (1, 2, 7), (1, 4, 32768), (2, 2, 16384)])
def test_hc_pre_norm_bit_exact(probe, orc, T, H, D):
    step(f"hc_pre_norm T={T} H={H} D={D}")
    rng = np.random.default_rng(T * 1000 + H * 10 + D)
    h = (rng.standard_normal((T, H, D)) * rng.choice([1e-3, 1.0, 40.0])).astype(np.float32)
    h[0, 0, : min(D, 3)] = -0.0
    mix = rng.standard_normal((T, 8)).astype(np.float32)
    w = rng.standard_normal(D).astype(np.float32)
    for ww in (None, w):
        want = orc.hc_pre_norm(h, mix, ww)
        x = torch.full((T, D), 7.0, dtype=torch.float32, device="cuda")
        probe.hc_pre_norm_async(dev(h), dev(mix), None if ww is None else dev(ww), x)
        probe.sync()
        assert np.array_equal(x.cpu().numpy().view(np.uint32), want.view(np.uint32)), ww is None


def test_hc_pre_norm_rejects_bad_arguments(probe):
    buf = torch.zeros(4 * 64 + 64, dtype=torch.float32, device="cuda")
    h = buf[:4 * 64].view(1, 4, 64)
    mix = torch.ones((1, 8), dtype=torch.float32, device="cuda")
    with pytest.raises(xl.XLError, match="overlaps"):
        probe.hc_pre_norm_async(h, mix, None, buf[192:256].view(1, 64))
    with pytest.raises(xl.XLError, match="epsilon"):
        probe.hc_pre_norm_async(h, mix, None, buf[256:].view(1, 64), eps=0.0)


def test_hc_post_rejects_overlap(probe):
    buf = torch.zeros(4 * 4 * 64 + 64, dtype=torch.float32, device="cuda")
    res = buf[64:64 + 4 * 64].view(1, 4, 64)
    post = torch.ones((1, 8), dtype=torch.float32, device="cuda")
    comb = torch.ones((1, 64), dtype=torch.float32, device="cuda")
    with pytest.raises(xl.XLError, match="overlaps"):
        probe.hc_post_async(buf[:64].view(1, 64), res, post, comb, buf[32:32 + 4 * 64].view(1, 4, 64))


def test_moe_block_composition(orc):
    """shared FFN -> routed layer with the shared row added last -> hc_post, all
    on one stream, against the oracle composition."""
    dim, ff, E, k, H = 1024, 512, 12, 6, 4
    step("MoE block: shared FFN + routed layer + hc_post")
    sig = (16, 16, 17)
    lane = xl.Lane(dim, ff, 1, E, types_map(1, E, sig[0], sig[2]), max_picks=8, swiglu_limit=7.0)
    try:
        lane.generate(seed=55)
        rng = np.random.default_rng(56)
        st = (13, 13, 14)
        g, u, dn = shared_mats(st, dim, 768, seed=57)
        x = (rng.standard_normal(dim) * 2.0).astype(np.float32)
        ids = rng.choice(E, k, replace=False).astype(np.int32)
        w = rng.random(k).astype(np.float32)
        res = rng.standard_normal((1, H, dim)).astype(np.float32)
        post = (rng.random((1, 8)) * 2).astype(np.float32)
        comb = rng.random((1, 64)).astype(np.float32)
        work = torch.empty(xl.shared_work_bytes(dim, 768, 1), dtype=torch.uint8, device="cuda")
        d_sh = torch.zeros((1, dim), dtype=torch.float32, device="cuda")
        d_moe = torch.zeros(dim, dtype=torch.float32, device="cuda")
        d_h2 = torch.zeros((1, H, dim), dtype=torch.float32, device="cuda")
        dx = dev(x)
        lane.shared_forward_async(st, dev(g), dev(u), dev(dn), 768, dx, d_sh, work)
        lane.layer_forward_async(0, dev(ids), dev(w), dx, d_moe, shared=d_sh)
        lane.hc_post_async(d_moe.view(1, dim), dev(res), dev(post), dev(comb), d_h2)
        lane.sync()
        sh = orc.expert32(st, g, u, dn, dim, 768, x, limit=7.0)
        rows = np.stack([orc.expert(sig, *orc.gen_expert(sig, 55, 0, int(e), dim, ff), dim, ff, x, limit=7.0)
                         for e in ids])
        moe = orc.combine(ids, w, rows, sh)
        assert max_rel(d_moe.cpu().numpy(), moe) < TOL
        want = orc.hc_post(moe[None], res, post, comb, dim, H, 1)
        assert max_rel(d_h2.cpu().numpy().reshape(-1), want.reshape(-1)) < TOL
        # hc_post itself is exact: on the device's own MoE row it matches bit for bit
        exact = orc.hc_post(d_moe.cpu().numpy()[None], res, post, comb, dim, H, 1)
        assert np.array_equal(d_h2.cpu().numpy().view(np.uint32), exact.view(np.uint32))
    finally:
        lane.close()
