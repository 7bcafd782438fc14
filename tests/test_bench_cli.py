"""bench.py without a GPU: the one-GPU refusal, the synthetic route
generators' invariants, and the algorithmic bytes the JSON line's `value`
divides by (config 1: 6 experts of IQ2_XXS gate/up 3,072 x 4,096 at 66 B and
IQ2_XS down 4,096 x 3,072 at 74 B per 256 weights, plus x in and y out; the
same formula at the real expert shape for config 6; config 5 adds the shared
expert's Q5_K gate/up and Q6_K down and hc_post's streams)."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("gen", [bench.routes, bench.zipf_routes])
def test_routes_are_distinct_picks_with_normalized_weights(gen):
    ids, w, x = gen(64, 7)
    assert ids.shape == (64, bench.K) and w.shape == (64, bench.K) and x.shape == (64, bench.DIM)
    for i in range(64):
        assert len(set(ids[i].tolist())) == bench.K
        assert ids[i].min() >= 0 and ids[i].max() < bench.E
        assert abs(float(w[i].astype(np.float64).sum()) - 1.0) < 1e-5 and np.all(w[i] > 0)
    ids2, w2, x2 = gen(64, 7)   # seeded
    assert np.array_equal(ids, ids2) and np.array_equal(w, w2) and np.array_equal(x, x2)


def test_topk_routes_take_the_largest_softmax_entries():
    rng = np.random.default_rng(7)
    ids, w, _ = bench.routes(4, 7)
    for i in range(4):
        logits = rng.standard_normal(bench.E).astype(np.float32)
        assert set(ids[i].tolist()) == set(np.argsort(-logits, kind="stable")[:bench.K].tolist())
        assert np.all(np.diff(w[i]) <= 0)   # descending probability


def test_algorithmic_bytes():
    assert bench.W_GU == 3_244_032 and bench.W_DN == 3_637_248
    assert bench.LAYER_BYTES == 60_784_640
    assert bench.expert_bytes((16, 16, 17)) * bench.K + 2 * bench.DIM * 4 == bench.LAYER_BYTES
    saved = bench.DIM, bench.FF
    try:
        bench.DIM, bench.FF = bench.REAL_DIM, bench.REAL_FF
        assert bench.expert_bytes((16, 16, 17)) * bench.K + 2 * bench.DIM * 4 == 56_995_840
    finally:
        bench.DIM, bench.FF = saved


def test_block_extra_bytes():
    # Q5_K: 176 B per 256 values, Q6_K: 210 B; gate and up 3,072 x 4,096, down 4,096 x 3,072
    assert bench.SHARED_T == (13, 13, 14)
    assert bench.dense_bytes(13, 3072, 4096) == 3072 * 16 * 176 == 8_650_752
    assert bench.dense_bytes(14, 4096, 3072) == 4096 * 12 * 210 == 10_321_920
    extra = 2 * 8_650_752 + 10_321_920 + 2 * 4 * 4096 * 4 + 72 * 4
    assert bench.block_extra_bytes() == extra == 27_754_784
    assert bench.LAYER_BYTES + extra == 88_539_424   # + the routed layer's: config 5's algorithmic bytes per step
