"""GPU parity of the device router (xl_route_async) with route.cpp:15-37 as the
oracle restates it (pinned bit for bit to the reference build on the CPU), and
of the routed layer / grouped calls against the oracle chain.

Ids must match exactly. The device's expf / log1pf are the device library's,
the oracle's glibc's: scores can differ in the last bits, so weights are held
to 2e-6 relative, and a token whose top-(k+1) keys lie within 1e-5 of each
other (where an ulp could legitimately reorder them) is excluded from the id
comparison; the tests assert such tokens stay rare.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.test_gpu_parity import TOL, dev, step, types_map

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def separable(lg, b, k):
    """Tokens whose k+1 largest keys are pairwise more than 1e-5 apart (relative),
    keys of bitwise-equal (logit, bias) pairs aside: those are equal on both sides."""
    bb = np.zeros(lg.shape[1], np.float32) if b is None else b
    sp = np.where(lg > 20, lg.astype(np.float64), np.log1p(np.exp(lg.astype(np.float64))))
    key = np.sqrt(sp) + bb.astype(np.float64)
    ok = np.ones(lg.shape[0], bool)
    for t in range(lg.shape[0]):
        order = np.argsort(-key[t], kind="stable")[:k + 1]
        for a, c in zip(order[:-1], order[1:]):
            same = lg[t, a] == lg[t, c] and bb[a] == bb[c]
            if not same and abs(key[t, a] - key[t, c]) <= 1e-5 * max(abs(key[t, c]), 1e-30):
                ok[t] = False
    return ok


@pytest.mark.parametrize("T,n,k,scale,spread,biased", [(64, 384, 6, 1.0, 1.0, False), (64, 384, 6, 2.5, 3.0, True),
                                                       (8, 4096, 8, 1.0, 10.0, True), (5, 16, 16, 0.5, 1.0, False),
                                                       (3, 1, 1, 1.0, 1.0, False)])
def test_route_matches_oracle(orc, T, n, k, scale, spread, biased):
    step(f"route T={T} n={n} k={k}")
    rng = np.random.default_rng(n + k + T)
    lg = (rng.standard_normal((T, n)) * spread).astype(np.float32)
    if n >= 8:
        lg[0, :6] = [25.0, 20.0, 19.5, -150.0, 3.0, 3.0]   # both softplus branches; an exact tie
    b = (rng.standard_normal(n) * 0.2).astype(np.float32) if biased else None
    want_ids, want_w = orc.route(lg, k, scale, b)
    lane = xl.Lane(256, 256, 1, 1, types_map(1, 1, 16, 16), max_picks=1)
    try:
        ids = torch.zeros((T, k), dtype=torch.int32, device="cuda")
        w = torch.zeros((T, k), dtype=torch.float32, device="cuda")
        lane.route_async(dev(lg), k, ids, w, scale=scale, bias=None if b is None else dev(b))
        lane.sync()
        got_ids, got_w = ids.cpu().numpy(), w.cpu().numpy()
    finally:
        lane.close()
    ok = separable(lg, b, k)
    assert ok.mean() > 0.95
    assert np.array_equal(got_ids[ok], want_ids[ok])
    np.testing.assert_allclose(got_w[ok], want_w[ok], rtol=2e-6, atol=1e-30)


def test_route_rejects_nonfinite():
    lane = xl.Lane(256, 256, 1, 1, types_map(1, 1, 16, 16), max_picks=1)
    try:
        lg = np.zeros((2, 8), np.float32); lg[1, 3] = np.inf
        ids = torch.zeros((2, 2), dtype=torch.int32, device="cuda"); w = torch.zeros((2, 2), device="cuda")
        lane.route_async(dev(lg), 2, ids, w)
        with pytest.raises(xl.XLError, match="non-finite"):
            lane.sync()
    finally:
        lane.close()


def oracle_layer(orc, types, seed, dim, ff, ids, w, x, shared=None):
    rows = []
    for e in ids:
        tt = tuple(int(v) for v in types[0, e])
        rows.append(orc.expert(tt, *orc.gen_expert(tt, seed, 0, int(e), dim, ff), dim, ff, x))
    return orc.combine(ids, w, np.stack(rows), shared)


def test_routed_layer_and_grouped(orc):
    # The router's ids and weights feed the layer kernels on the device; the
    # result is the oracle chain on the oracle's own routing.
    dim, ff, E, k, T = 1024, 512, 32, 6, 12
    step("routed layer + grouped")
    rng = np.random.default_rng(12)
    types = types_map(1, E, 16, 17)
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=8, max_tokens=16)
    try:
        lane.generate(seed=21)
        lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
        b = (rng.standard_normal(E) * 0.1).astype(np.float32)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        ids, w = orc.route(lg, k, 1.5, b)
        assert separable(lg, b, k).all()
        d_lg, d_b, d_x = dev(lg), dev(b), dev(x)
        out = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        for t in range(T):
            lane.layer_forward_routed_async(0, d_lg[t], k, d_x[t], out[t], scale=1.5, bias=d_b)
        lane.sync()
        got = out.cpu().numpy()
        gout = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        lane.grouped_forward_routed_async(0, d_lg, k, d_x, gout, scale=1.5, bias=d_b)
        lane.sync()
        ggot = gout.cpu().numpy()
        for t in range(T):
            want = oracle_layer(orc, types, 21, dim, ff, ids[t], w[t], x[t])
            assert max_rel(got[t], want) < TOL, (t, max_rel(got[t], want))
            assert max_rel(ggot[t], want) < TOL, (t, max_rel(ggot[t], want))
    finally:
        lane.close()


@pytest.mark.parametrize("dim,ff,E,k,kind", [(4096, 3072, 384, 6, "iq2"), (4096, 3072, 384, 1, "iq2"),
                                             (4096, 3072, 64, 6, "iq1"), (1024, 512, 600, 4, "iq2"),
                                             (1024, 512, 40, 3, "mixed")])
def test_routed_one_launch_matches_router_then_layer(dim, ff, E, k, kind):
    # Where the streaming kernel has the layer and E <= 512, the routed call is
    # one launch that routes in its prologue (every wave from the logits); it
    # must give the bits of the router kernel followed by the layer call on its
    # ids and weights (E = 600: the two-launch path itself). Ties included: a
    # few logits repeat exactly.
    step(f"routed one launch dim={dim} ff={ff} E={E} k={k} {kind}")
    rng = np.random.default_rng(E + k)
    if kind == "mixed":
        types = np.repeat(rng.choice([16, 17, 29], size=(1, E)).astype(np.int32)[..., None], 3, axis=-1)
    else:
        t = (16, 17) if kind == "iq2" else (29, 29)
        types = types_map(1, E, t[0], t[1])
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=8)
    try:
        lane.generate(seed=33)
        T = 6
        lg = (rng.standard_normal((T, E)) * 2).astype(np.float32)
        lg[:, 5] = lg[:, 3]   # an exact tie of keys (the lower index wins)
        b = (rng.standard_normal(E) * 0.1).astype(np.float32)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        d_lg, d_b, d_x = dev(lg), dev(b), dev(x)
        one = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        two = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        ids = torch.zeros((T, k), dtype=torch.int32, device="cuda")
        w = torch.zeros((T, k), dtype=torch.float32, device="cuda")
        lane.route_async(d_lg, k, ids, w, scale=1.5, bias=d_b)
        for t in range(T):
            lane.layer_forward_routed_async(0, d_lg[t], k, d_x[t], one[t], scale=1.5, bias=d_b)
            lane.layer_forward_async(0, ids[t], w[t], d_x[t], two[t])
        lane.sync()
        assert np.array_equal(one.cpu().numpy().view(np.uint32), two.cpu().numpy().view(np.uint32))
        # the routed calls routed inside their launch where one exists (E <= 512),
        # so the comparison above is the one launch against the two calls
        counts = lane.launch_counts()
        assert counts["routed"] == (T if E <= 512 else 0), counts
        assert counts["stream"] == (T if E <= 512 else 2 * T), counts
    finally:
        lane.close()
