"""GPU parity of the pre-normed layer call (xl_layer_forward_prenorm_async): the
MoE layer of one token whose input is the hyper-connection pre + RMS norm of the
previous hidden (hip_backend.cpp:629 k4::hc_pre_norm, then the layer). With one
stream and a streaming-kernel layer it is one launch that normalizes in every
workgroup's prologue; otherwise the pre-norm kernel and the layer. Either way x
and the layer output must equal, bit for bit, those of xl_hc_pre_norm_async
followed by xl_layer_forward_async, and x must equal the oracle's pre-norm
(oracle/xl_oracle.c orc_hc_pre_norm, pinned to sycl/hc/core.hpp:74-80).
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.test_gpu_parity import dev, kind_types, route, step

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

E = 24
SHAPES = [(4096, 3072, 6), (4096, 3072, 1), (1024, 512, 16), (256, 768, 12), (5120, 2304, 6), (5120, 2304, 2)]


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def both(lane, ids, w, h, mix, nw, shared=None, eps=1e-6):
    """(x, out) of the one call and of the two calls, on one stream."""
    dim = h.shape[-1]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        x1 = torch.full((dim,), float("nan"), dtype=torch.float32, device="cuda")
        y1 = torch.full((dim,), float("nan"), dtype=torch.float32, device="cuda")
        x2, y2 = x1.clone(), y1.clone()
        lane.layer_forward_prenorm_async(0, ids, w, h, mix, nw, x1, y1, eps=eps, shared=shared, stream=s.cuda_stream)
        lane.hc_pre_norm_async(h.view(1, -1, dim), mix.view(1, 8), nw, x2.view(1, dim), eps=eps,
                               stream=s.cuda_stream)
        lane.layer_forward_async(0, ids, w, x2, y2, shared=shared, stream=s.cuda_stream)
    lane.sync(s.cuda_stream)
    torch.cuda.synchronize()
    return x1, y1, x2, y2


@pytest.mark.parametrize("kind", ["iq2", "iq1", "mixed"])
@pytest.mark.parametrize("dim,ff,k", SHAPES)
def test_prenorm_layer_matches_norm_then_layer(orc, kind, dim, ff, k):
    step(f"pre-normed layer {kind} dim={dim} ff={ff} k={k}")
    rng = np.random.default_rng(dim * 7 + ff + k)
    lane = xl.Lane(dim, ff, 1, E, kind_types(kind, E), max_picks=16)
    try:
        lane.generate(seed=57)
        for trial in range(3):
            ids, w = route(rng.standard_normal(E).astype(np.float32), k)
            h = (rng.standard_normal(dim) * (1 + 3 * trial)).astype(np.float32)
            mix = np.zeros(8, np.float32)
            mix[0] = (0.5, 1.0, -1.25)[trial]
            nw = None if trial == 1 else (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
            shared = rng.standard_normal(dim).astype(np.float32) if trial == 2 else None
            x1, y1, x2, y2 = both(lane, dev(ids), dev(w), dev(h).view(1, dim), dev(mix),
                                  None if nw is None else dev(nw), None if shared is None else dev(shared))
            assert np.array_equal(bits(x1), bits(x2)), trial
            assert np.array_equal(bits(y1), bits(y2)), trial
            want_x = orc.hc_pre_norm(h.reshape(1, 1, dim), mix.reshape(1, 8), nw)[0]
            assert np.array_equal(bits(x1), want_x.view(np.uint32)), trial
            assert np.all(np.isfinite(y1.cpu().numpy()))
            # the pre-normed call normalized inside its one launch (not the two-call fallback)
            assert lane.launch_counts()["prenorm"] == trial + 1
    finally:
        lane.close()


def test_prenorm_layer_several_streams(orc):
    # H = 2: the pre-norm kernel and then the layer, bit-identical all the same
    step("pre-normed layer, two streams")
    rng = np.random.default_rng(5)
    lane = xl.Lane(4096, 3072, 1, E, kind_types("iq2", E), max_picks=8)
    try:
        lane.generate(seed=57)
        ids, w = route(rng.standard_normal(E).astype(np.float32), 6)
        h = rng.standard_normal((2, 4096)).astype(np.float32)
        mix = np.zeros(8, np.float32)
        mix[:2] = (0.75, -0.5)
        nw = (1 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
        x1, y1, x2, y2 = both(lane, dev(ids), dev(w), dev(h), dev(mix), dev(nw))
        assert np.array_equal(bits(x1), bits(x2))
        assert np.array_equal(bits(y1), bits(y2))
        want_x = orc.hc_pre_norm(h.reshape(1, 2, 4096), mix.reshape(1, 8), nw)[0]
        assert np.array_equal(bits(x1), want_x.view(np.uint32))
    finally:
        lane.close()


def test_prenorm_layer_rejects_bad_arguments():
    step("pre-normed layer: argument checks")
    lane = xl.Lane(1024, 512, 1, E, kind_types("iq2", E), max_picks=8)
    try:
        lane.generate(seed=57)
        ids, w = dev(np.arange(6, dtype=np.int32)), dev(np.full(6, 1 / 6, np.float32))
        buf = torch.zeros(4 * 1024, dtype=torch.float32, device="cuda")
        h, x, out = buf[:1024].view(1, 1024), buf[1024:2048], buf[2048:3072]
        mix = torch.zeros(8, dtype=torch.float32, device="cuda")
        mix[0] = 1.0
        for bad in (dict(x=buf[512:1536]),                 # x overlaps h
                    dict(out=buf[:1024]),                  # out is h
                    dict(out=buf[1024:2048]),              # out is x
                    dict(eps=0.0), dict(eps=float("inf"))):
            a = dict(x=x, out=out, eps=1e-6)
            a.update(bad)
            with pytest.raises(xl.XLError):
                lane.layer_forward_prenorm_async(0, ids, w, h, mix, None, a["x"], a["out"], eps=a["eps"])
        with pytest.raises(xl.XLError):   # five streams
            lane.layer_forward_prenorm_async(0, ids, w, torch.zeros((5, 1024), device="cuda"), mix, None, x, out)
        lane.sync()
    finally:
        lane.close()
