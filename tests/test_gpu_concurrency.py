"""Calls on one context from two streams, and the single-launch kernels'
launch counters across their 2^32 wrap.

Every call on a context waits on the GPU for the context's previous call when
that one ran on another stream (the calls share the workspace, the h exchange
buffers and the counters), so interleaving two streams without host
synchronization must give, call by call, the bits serial calls give. The
counters (the all-types kernel's epoch, the streaming kernel's launch count)
are set just below 2^32 and stepped over the wrap: every launch must still
match the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.test_gpu_parity import TOL, dev, route, step, types_map

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

DIM, FF, E, K, SEED = 4096, 3072, 16, 6, 0x2517


def routes(n, seed):
    rng = np.random.default_rng(seed)
    ids = np.zeros((n, K), np.int32)
    w = np.zeros((n, K), np.float32)
    for i in range(n):
        ids[i], w[i] = route(rng.standard_normal(E).astype(np.float32), K)
    return ids, w, rng.standard_normal((n, DIM)).astype(np.float32)


def oracle_layer(orc, sig, ids, w, x):
    rows = [orc.expert(sig, *orc.gen_expert(sig, SEED, 0, int(e), DIM, FF), DIM, FF, x) for e in ids]
    return orc.combine(ids, w, np.stack(rows))


@pytest.mark.parametrize("path,sig", [("4", (16, 16, 17)), ("4", (29, 29, 29)), ("3", (16, 16, 17)),
                                      ("3", (29, 29, 29))])
def test_two_streams_one_context(orc, monkeypatch, path, sig):
    monkeypatch.setenv("XL_LAYER_PATH", path)
    step(f"two streams: XL_LAYER_PATH={path} sig={sig}")
    lane = xl.Lane(DIM, FF, 1, E, types_map(1, E, sig[0], sig[2]), max_picks=8)
    try:
        lane.generate(SEED)
        n = 24
        ids, w, x = routes(n, SEED + int(path))
        serial = np.stack([lane.layer_forward(0, ids[i], w[i], x[i]) for i in range(n)])
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        d_ids, d_w, d_x = dev(ids), dev(w), dev(x)
        out = torch.zeros((n, DIM), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        for rep in range(2):
            for i in range(n):   # alternate streams, no host synchronization in between
                s = (sa if i % 2 == 0 else sb).cuda_stream
                lane.layer_forward_async(0, d_ids[i], d_w[i], d_x[i], out[i], stream=s)
            lane.sync(sa.cuda_stream)
            lane.sync(sb.cuda_stream)
            got = out.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), serial.view(np.uint32)), rep
        for i in (0, n - 1):
            assert max_rel(serial[i], oracle_layer(orc, sig, ids[i], w[i], x[i])) < TOL
    finally:
        lane.close()


@pytest.mark.parametrize("path", ["4", "3"])
@pytest.mark.parametrize("start", [0xFFFFFFFD, 0xFFFFFFFE, 1])
def test_launch_counter_wrap(orc, monkeypatch, path, start):
    # The counters set to either parity near the wrap, and set back to a count
    # whose epochs earlier launches already used (start 1 after five launches):
    # every later launch must still compute its own call, bit for bit.
    monkeypatch.setenv("XL_LAYER_PATH", path)
    step(f"counter wrap: XL_LAYER_PATH={path} start={start:#x}")
    sig = (16, 16, 17)
    lane = xl.Lane(DIM, FF, 1, E, types_map(1, E, sig[0], sig[2]), max_picks=8)
    try:
        lane.generate(SEED)
        ids, w, x = routes(6, SEED + 7)
        want = [lane.layer_forward(0, ids[i], w[i], x[i]) for i in range(6)]   # counters far from the wrap
        lane.debug_set_launch_count(start)
        for i in (5, 4, 3, 2, 1, 0):   # other inputs than the last launches: stale words would show
            got = lane.layer_forward(0, ids[i], w[i], x[i])
            assert np.array_equal(got.view(np.uint32), want[i].view(np.uint32)), i
        assert max_rel(want[4], oracle_layer(orc, sig, ids[4], w[4], x[4])) < TOL
        counts = lane.launch_counts()
        assert counts["stream" if path == "4" else "alltypes"] == 12, counts
    finally:
        lane.close()
