"""GPU parity of the grouped path (xl_grouped_forward): T tokens with k picks
each must give what T per-token layer calls give (the reference's per-token
warm_compute_many + fixed-order combine, engine/strata/warm/runtime.hpp:13,
runtime.cpp:180-188): the oracle within the 1e-3 max-relative bar, and bit
identity run to run.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.test_gpu_parity import TOL, dev, route, step, types_map

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def token_routes(rng, T, E, k, skew=None):
    """Per token: k distinct ids from the softmax of N(0,1) logits (plus a
    per-expert bias `skew` that piles picks onto a few experts)."""
    ids = np.zeros((T, k), np.int32)
    w = np.zeros((T, k), np.float32)
    for t in range(T):
        logits = rng.standard_normal(E).astype(np.float32)
        if skew is not None:
            logits = logits + skew
        ids[t], w[t] = route(logits, k)
    return ids, w


def oracle_out(orc, types, seed, dim, ff, ids, w, x, shared=None):
    cache = {}
    out = np.zeros((ids.shape[0], dim), np.float32)
    for t in range(ids.shape[0]):
        rows = []
        for e in ids[t]:
            tt = tuple(int(v) for v in types[0, e])
            if int(e) not in cache:
                cache[int(e)] = orc.gen_expert(tt, seed, 0, int(e), dim, ff)
            rows.append(orc.expert(tt, *cache[int(e)], dim, ff, x[t]))
        out[t] = orc.combine(ids[t], w[t], np.stack(rows), None if shared is None else shared[t])
    return out


@pytest.mark.parametrize("dim,ff,E,T,k,skewed", [(4096, 3072, 24, 24, 6, False), (4096, 3072, 24, 20, 6, True),
                                                 (1024, 512, 8, 40, 8, True), (256, 768, 6, 1, 1, False),
                                                 (1024, 512, 16, 33, 3, False)])
def test_grouped_vs_oracle_and_layer_calls(orc, dim, ff, E, T, k, skewed, monkeypatch):
    # skewed: most picks land on a few experts, so those get several 16-pair
    # tasks. XL_GROUPED_PATH=2: the MFMA kernels run or the call fails.
    step(f"grouped dim={dim} ff={ff} E={E} T={T} k={k} skewed={skewed}")
    rng = np.random.default_rng(dim + 3 * T + k)
    types = types_map(1, E, 16, 17)
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=8, max_tokens=64)
    try:
        lane.generate(seed=5)
        skew = np.where(np.arange(E) < 3, 4.0, 0.0).astype(np.float32) if skewed else None
        ids, w = token_routes(rng, T, E, k, skew)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        shared = rng.standard_normal((T, dim)).astype(np.float32)
        for sh in (None, shared):
            got = lane.grouped_forward(0, ids, w, x, sh)
            again = lane.grouped_forward(0, ids, w, x, sh)
            assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
            want = oracle_out(orc, types, 5, dim, ff, ids, w, x, sh)
            assert max_rel(got, want) < TOL, max_rel(got, want)
            per = np.stack([lane.layer_forward(0, ids[t], w[t], x[t], None if sh is None else sh[t]) for t in range(T)])
            assert max_rel(got, per) < TOL, max_rel(got, per)
    finally:
        lane.close()


@pytest.mark.parametrize("T", [16, 17, 33])
def test_grouped_task_boundaries(orc, T, monkeypatch):
    """Expert 0 picked by every token: exactly one full 16-pair task (T = 16),
    a full task plus a one-pair task (17), two full tasks plus one (33); the
    second pick spreads over experts 1..3. Against per-token layer calls and
    the oracle."""
    dim, ff, E, k = 1024, 512, 4, 2
    step(f"grouped task boundaries T={T}")
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    types = types_map(1, E, 16, 17)
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=k, max_tokens=64)
    try:
        lane.generate(seed=9)
        rng = np.random.default_rng(T)
        ids = np.stack([np.zeros(T, np.int32), (1 + np.arange(T) % 3).astype(np.int32)], axis=1)
        w = rng.random((T, k)).astype(np.float32)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        got = lane.grouped_forward(0, ids, w, x)
        per = np.stack([lane.layer_forward(0, ids[t], w[t], x[t]) for t in range(T)])
        assert max_rel(got, per) < TOL, max_rel(got, per)
        pick = [0, 15, T - 1]
        want = oracle_out(orc, types, 9, dim, ff, ids[pick], w[pick], x[pick], None)
        assert max_rel(got[pick], want) < TOL, max_rel(got[pick], want)
    finally:
        lane.close()


def test_grouped_async_and_other_types(orc):
    # Device pointers on a caller stream; a layer whose types the MFMA kernels do
    # not take (IQ1_M) runs one layer call per token and matches those calls bit
    # for bit.
    dim, ff, E, T, k = 1024, 512, 8, 12, 4
    step("grouped async + IQ1_M per-token path")
    rng = np.random.default_rng(44)
    types = np.concatenate([types_map(1, E, 16, 17), types_map(1, E, 29, 29)], axis=0)
    lane = xl.Lane(dim, ff, 2, E, types, max_picks=4, max_tokens=16)
    try:
        lane.generate(seed=8)
        ids, w = token_routes(rng, T, E, k)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        s = torch.cuda.Stream()
        for layer in (0, 1):
            out = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
            with torch.cuda.stream(s):
                d_ids, d_w, d_x = dev(ids), dev(w), dev(x)
            lane.grouped_forward_async(layer, d_ids, d_w, d_x, out, stream=s.cuda_stream)
            lane.sync(s.cuda_stream)
            got = out.cpu().numpy()
            per = np.stack([lane.layer_forward(layer, ids[t], w[t], x[t]) for t in range(T)])
            if layer == 1:
                assert np.array_equal(got.view(np.uint32), per.view(np.uint32))
            else:
                assert max_rel(got, per) < TOL
            tt = tuple(int(v) for v in types[layer, 0])
            want = np.stack([orc.combine(ids[t], w[t], np.stack([orc.expert(tt, *orc.gen_expert(tt, 8, layer, int(e), dim, ff),
                                                                            dim, ff, x[t]) for e in ids[t]]))
                             for t in range(3)])
            assert max_rel(got[:3], want) < TOL
    finally:
        lane.close()


def test_grouped_bad_id_and_limits(monkeypatch):
    dim, ff, E = 1024, 512, 4
    step("grouped bad id / limits")
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    lane = xl.Lane(dim, ff, 1, E, types_map(1, E, 16, 17), max_picks=2, max_tokens=4)
    try:
        lane.generate(2)
        x = np.ones((2, dim), np.float32)
        with pytest.raises(xl.XLError, match="max_tokens"):
            lane.grouped_forward(0, np.zeros((5, 1), np.int32), np.ones((5, 1), np.float32), np.ones((5, dim), np.float32))
        with pytest.raises(xl.XLError, match="duplicate"):
            lane.grouped_forward(0, np.array([[1, 1], [0, 2]], np.int32), np.full((2, 2), 0.5, np.float32), x)
        out = torch.zeros((2, dim), dtype=torch.float32, device="cuda")
        lane.grouped_forward_async(0, dev(np.array([[1, 99], [0, 2]], np.int32)), dev(np.full((2, 2), 0.5, np.float32)),
                                   dev(x), out)
        with pytest.raises(xl.XLError, match="expert id"):
            lane.sync()
    finally:
        lane.close()
    with pytest.raises(xl.XLError, match="XL_GROUPED_PATH=2"):
        ctx2 = xl.Lane(dim, ff, 1, E, types_map(1, E, 29, 29), max_picks=2, max_tokens=4)
        try:
            ctx2.generate(2)
            ctx2.grouped_forward(0, np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32), np.ones((1, dim), np.float32))
        finally:
            ctx2.close()
    ctx0 = xl.Lane(dim, ff, 1, E, types_map(1, E, 16, 17), max_picks=2)
    try:
        ctx0.generate(2)
        with pytest.raises(xl.XLError, match="max_tokens = 0"):
            ctx0.grouped_forward(0, np.zeros((1, 1), np.int32), np.ones((1, 1), np.float32), np.ones((1, dim), np.float32))
    finally:
        ctx0.close()


def test_grouped_unaligned_out_and_shared(monkeypatch):
    # out and shared 4 bytes off a 16-byte boundary take the one-column combine;
    # it must equal the four-column combine of aligned buffers bit for bit
    step("grouped combine: unaligned out / shared")
    rng = np.random.default_rng(77)
    E, T, k, dim = 16, 12, 6, 1024
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    lane = xl.Lane(dim, 512, 1, E, types_map(1, E, 16, 17), max_picks=8, max_tokens=64)
    try:
        lane.generate(seed=5)
        ids, w = token_routes(rng, T, E, k)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        sh = rng.standard_normal((T, dim)).astype(np.float32)
        d_ids, d_w, d_x = dev(ids), dev(w), dev(x)
        a_sh, a_out = dev(sh), torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        u_sh_buf = torch.zeros(T * dim + 1, dtype=torch.float32, device="cuda")
        u_out_buf = torch.zeros(T * dim + 1, dtype=torch.float32, device="cuda")
        u_sh, u_out = u_sh_buf[1:].view(T, dim), u_out_buf[1:].view(T, dim)
        assert u_sh.data_ptr() % 16 == 4 and u_out.data_ptr() % 16 == 4
        u_sh.copy_(a_sh)
        lane.grouped_forward_async(0, d_ids, d_w, d_x, a_out, shared=a_sh)
        lane.grouped_forward_async(0, d_ids, d_w, d_x, u_out, shared=u_sh)
        lane.sync()
        assert np.array_equal(a_out.cpu().numpy().view(np.uint32), u_out.cpu().numpy().view(np.uint32))
    finally:
        lane.close()
