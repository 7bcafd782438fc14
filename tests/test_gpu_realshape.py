"""The DeepSeek-V4.1 expert shape, d_model 5120 x d_ff 2304
(engine/strata/fixtures/moe/cpu_lane_fixture.cpp:17; the reference's own checks
run K = 2304 / 5120, warm/grouped_check.hpp:89, warm/expert_check.cpp:144), on
every path: the streaming kernel's 5120 x 2304 instances (IQ2, IQ1_M and
mixed-type layers, up to 6 picks) and the all-types kernel (more picks, or
forced) with their parity traces, the separate launches, the per32 mode, the
grouped MFMA kernels, and a weight pack in the reference's layout loaded
through xl_bank_load_pack.

Bars as everywhere: Q8_K bytes and block integers of the kernel's own data
bit-exact, outputs within max relative error 1e-3 of the oracle, reruns
bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.packs import write_pack
from tests.test_gpu_grouped import token_routes
from tests.test_gpu_parity import TOL, dev, route, step, types_map
from tests.test_gpu_trace import check_pick, layer_types, zeros

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

DIM, FF, SEED = 5120, 2304, 0x5120


@pytest.mark.parametrize("kind,k,path,kernel,lim", [
    ("iq2", 6, "1", 1, 0.0), ("iq1", 6, "1", 1, 0.0), ("mixed", 6, "1", 1, 10.0), ("iq2", 1, "1", 1, 10.0),
    ("iq2", 2, "1", 1, 0.0), ("mixed", 3, "1", 1, 0.0), ("mixed", 8, "1", 3, 0.0), ("iq2", 6, "3", 3, 10.0),
    ("iq1", 6, "3", 3, 0.0)])
def test_real_shape_layer(orc, monkeypatch, kind, k, path, kernel, lim):
    E = 12
    types = layer_types(kind, E)
    step(f"real shape {DIM}x{FF} layer {kind} k={k} path={path} lim={lim}")
    monkeypatch.setenv("XL_LAYER_PATH", path)
    lane = xl.Lane(DIM, FF, 1, E, types, max_picks=8, swiglu_limit=lim)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(k + len(kind))
        ids, w = route(rng.standard_normal(E).astype(np.float32), k)
        x = rng.standard_normal(DIM).astype(np.float32)
        rows, mats = [], []
        for e in ids:
            sig = tuple(int(v) for v in types[0, e])
            mats.append(orc.gen_expert(sig, SEED, 0, int(e), DIM, FF))
            rows.append(orc.expert(sig, *mats[-1], DIM, FF, x, limit=lim))
        want = orc.combine(ids, w, np.stack(rows))
        got = lane.layer_forward(0, ids, w, x)
        assert max_rel(got, want) < TOL, max_rel(got, want)
        assert np.array_equal(got.view(np.uint32), lane.layer_forward(0, ids, w, x).view(np.uint32))
        # the launch's own Q8_K bytes and block integers
        nbx, nbh = DIM // 256, FF // 256
        rec = 2 * FF * nbx + DIM * nbh
        out = zeros(DIM, torch.float32)
        q8x, q8h = zeros(nbx * 292, torch.uint8), zeros(k * nbh * 292, torch.uint8)
        h, ints = zeros(k * FF, torch.float32), zeros(k * rec, torch.int32)
        torch.cuda.synchronize()
        assert lane.layer_trace_async(0, dev(ids), dev(w), dev(x), out, q8x, q8h, h, ints) == kernel
        lane.sync()
        want_q8x = orc.quantize(x)
        assert np.array_equal(q8x.cpu().numpy(), want_q8x.view(np.uint8))
        h, q8h, ints = h.cpu().numpy().reshape(k, FF), q8h.cpu().numpy().reshape(k, -1), ints.cpu().numpy().reshape(k, rec)
        for i, e in enumerate(ids):
            sig = tuple(int(v) for v in types[0, e])
            check_pick(orc, sig, mats[i], DIM, FF, want_q8x, h[i], q8h[i], ints[i], f"pick {i} expert {e} {sig}")
        assert np.array_equal(out.cpu().numpy().view(np.uint32), got.view(np.uint32))
        # separate launches (the fallback) on the same layer
        monkeypatch.setenv("XL_LAYER_PATH", "0")
        sep = xl.Lane(DIM, FF, 1, E, types, max_picks=8, swiglu_limit=lim)
        try:
            sep.generate(SEED)
            got0 = sep.layer_forward(0, ids, w, x)
            assert max_rel(got0, want) < TOL, max_rel(got0, want)
        finally:
            sep.close()
    finally:
        lane.close()


def test_real_shape_per32(orc):
    E, k = 8, 6
    types = layer_types("mixed", E)
    step(f"real shape per32 k={k}")
    lane = xl.Lane(DIM, FF, 1, E, types, max_picks=8)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(32)
        ids, w = route(rng.standard_normal(E).astype(np.float32), k)
        x = rng.standard_normal(DIM).astype(np.float32)
        y, out = lane.layer_forward_per32(0, ids, x, weights=w)
        rows = []
        for e in ids:
            sig = tuple(int(v) for v in types[0, e])
            rows.append(orc.expert32(sig, *orc.gen_expert(sig, SEED, 0, int(e), DIM, FF), DIM, FF, x))
        for i in range(k):
            assert max_rel(y[i], rows[i]) < TOL, (i, max_rel(y[i], rows[i]))
        assert np.array_equal(out.view(np.uint32), orc.combine(ids, w, y).view(np.uint32))
    finally:
        lane.close()


def test_real_shape_grouped(orc, monkeypatch):
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    E, T, k = 16, 24, 6
    types = types_map(1, E, 16, 17)
    step(f"real shape grouped T={T} E={E} k={k}")
    lane = xl.Lane(DIM, FF, 1, E, types, max_picks=8, max_tokens=32)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(24)
        ids, w = token_routes(rng, T, E, k)
        x = rng.standard_normal((T, DIM)).astype(np.float32)
        got = lane.grouped_forward(0, ids, w, x)
        assert np.array_equal(got.view(np.uint32), lane.grouped_forward(0, ids, w, x).view(np.uint32))
        per = np.stack([lane.layer_forward(0, ids[t], w[t], x[t]) for t in range(T)])
        assert max(max_rel(got[t], per[t]) for t in range(T)) < TOL
        cache = {int(e): orc.gen_expert((16, 16, 17), SEED, 0, int(e), DIM, FF) for e in np.unique(ids[:2])}
        for t in range(2):
            rows = [orc.expert((16, 16, 17), *cache[int(e)], DIM, FF, x[t]) for e in ids[t]]
            assert max_rel(got[t], orc.combine(ids[t], w[t], np.stack(rows))) < TOL
        # the MFMA kernels' own Q8_K bytes and block integers for the first token's pairs
        nbx, nbh, P = DIM // 256, FF // 256, T * k
        rec = 2 * FF * nbx + DIM * nbh
        out = zeros((T, DIM), torch.float32)
        q8x, q8h = zeros(T * nbx * 292, torch.uint8), zeros(P * nbh * 292, torch.uint8)
        h, ints = zeros(P * FF, torch.float32), zeros(P * rec, torch.int32)
        torch.cuda.synchronize()
        lane.grouped_trace_async(0, dev(ids), dev(w), dev(x), out, q8x, q8h, h, ints)
        lane.sync()
        q8x = q8x.cpu().numpy().reshape(T, -1)
        h, q8h, ints = h.cpu().numpy().reshape(P, FF), q8h.cpu().numpy().reshape(P, -1), ints.cpu().numpy().reshape(P, rec)
        want_q8x = orc.quantize(x[0])
        assert np.array_equal(q8x[0], want_q8x.view(np.uint8))
        for i, e in enumerate(ids[0]):
            check_pick(orc, (16, 16, 17), cache[int(e)], DIM, FF, want_q8x, h[i], q8h[i], ints[i], f"pair {i}")
    finally:
        lane.close()


def test_real_shape_pack(orc, tmp_path):
    E = 4
    sigs = [(29, 29, 29), (16, 16, 17)]
    step("real shape pack")
    p = write_pack(str(tmp_path / "pack"), orc, sigs, DIM, FF, E, seed=77)
    meta = xl.pack_meta(p)
    assert (meta["dim"], meta["ff"]) == (DIM, FF)
    types = xl.pack_types(p, 0, len(sigs), E)
    lane = xl.Lane(DIM, FF, len(sigs), E, types, max_picks=4)
    try:
        lane.load_pack(p)
        for l, sig in enumerate(sigs):
            for r in range(3):
                n, kk = (FF, DIM) if r < 2 else (DIM, FF)
                assert np.array_equal(lane.download(l, E - 1, r), orc.gen_matrix(sig[r], 77, l, E - 1, r, n, kk))
            ids = np.array([3, 0, 2], np.int32)
            w = np.array([0.5, 0.3, 0.2], np.float32)
            x = np.random.default_rng(l).standard_normal(DIM).astype(np.float32)
            rows = [orc.expert(sig, *orc.gen_expert(sig, 77, l, int(e), DIM, FF), DIM, FF, x) for e in ids]
            got = lane.layer_forward(l, ids, w, x)
            assert max_rel(got, orc.combine(ids, w, np.stack(rows))) < TOL
    finally:
        lane.close()
