"""The SwiGLU limit (model_meta.hpp:34 `lim`, the pack's swiglu_limit) on every
layer path: with lim > 0 the gate is clamped to <= lim and the up projection to
[-lim, lim] before SiLU(g) * u (q8k_core.hpp:92-95). Each path is held to the
oracle chain with the same limit, within max-rel 1e-3; the limit is chosen so
that it changes the output by far more than the tolerance.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu
TOL = 1e-3
LIM = 7.0
SEED = 4242

torch = pytest.importorskip("torch")


def step(msg):
    print(f"[gpu-step] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def routes(rng, E, k):
    ids = rng.choice(E, k, replace=False).astype(np.int32)
    return ids, (rng.random(k).astype(np.float32) + 0.1)


@pytest.mark.parametrize("dim,ff,sig", [(4096, 3072, (16, 16, 17)), (1024, 512, (29, 29, 29)),
                                        (1024, 512, (17, 17, 16))])
def test_layer_paths_with_limit(orc, dim, ff, sig, monkeypatch):
    step(f"swiglu limit {LIM}: layer paths dim={dim} ff={ff} sig={sig}")
    E, k = 16, 6
    rng = np.random.default_rng(dim + ff + sig[0])
    types = np.zeros((1, E, 3), np.int32)
    types[..., 0], types[..., 1], types[..., 2] = sig
    lanes = {}
    try:
        for path in ("1", "3", "0"):
            monkeypatch.setenv("XL_LAYER_PATH", path)
            lanes[path] = xl.Lane(dim, ff, 1, E, types, max_picks=8, swiglu_limit=LIM)
            lanes[path].generate(seed=SEED)
        mats = {e: orc.gen_expert(sig, SEED, 0, e, dim, ff) for e in range(E)}
        for trial in range(2):
            ids, w = routes(rng, E, k)
            x = (rng.standard_normal(dim) * 2.0).astype(np.float32)
            want = orc.combine(ids, w, np.stack([orc.expert(sig, *mats[int(e)], dim, ff, x, limit=LIM) for e in ids]))
            free = orc.combine(ids, w, np.stack([orc.expert(sig, *mats[int(e)], dim, ff, x) for e in ids]))
            assert max_rel(free, want) > 100 * TOL   # the limit bites
            for path, lane in lanes.items():
                got = lane.layer_forward(0, ids, w, x)
                assert max_rel(got, want) < TOL, (path, trial, max_rel(got, want))
            # per32 mode with the same limit
            y32, _ = lanes["1"].layer_forward_per32(0, ids, x)
            for i, e in enumerate(ids):
                assert max_rel(y32[i], orc.expert32(sig, *mats[int(e)], dim, ff, x, limit=LIM)) < TOL, (trial, i)
    finally:
        for lane in lanes.values():
            lane.close()


def test_grouped_with_limit(orc, monkeypatch):
    dim, ff, E, T, k = 1024, 512, 12, 20, 4
    sig = (16, 16, 17)
    step(f"swiglu limit {LIM}: grouped MFMA path T={T}")
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    types = np.zeros((1, E, 3), np.int32)
    types[..., 0], types[..., 1], types[..., 2] = sig
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=k, max_tokens=T, swiglu_limit=LIM)
    try:
        lane.generate(seed=SEED)
        rng = np.random.default_rng(7)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
        w = rng.random((T, k)).astype(np.float32)
        x = (rng.standard_normal((T, dim)) * 2.0).astype(np.float32)
        got = lane.grouped_forward(0, ids, w, x)
        mats = {e: orc.gen_expert(sig, SEED, 0, e, dim, ff) for e in range(E)}
        for t in range(T):
            rows = np.stack([orc.expert(sig, *mats[int(e)], dim, ff, x[t], limit=LIM) for e in ids[t]])
            assert max_rel(got[t], orc.combine(ids[t], w[t], rows)) < TOL, t
    finally:
        lane.close()


def test_limit_rejected_when_not_finite():
    types = np.full((1, 2, 3), 16, np.int32)
    with pytest.raises(xl.XLError):
        xl.Lane(256, 256, 1, 2, types, max_picks=2, swiglu_limit=float("nan"))
