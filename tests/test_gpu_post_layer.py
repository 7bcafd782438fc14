"""GPU parity of the layer call with the hyper-connection post after it
(xl_layer_forward_post_async): the MoE layer of one token (shared row added
last) and hc_post of its output (hip_backend.cpp:635-711, then :777
k4::hc_post). With a streaming-kernel layer it is one launch whose combine
applies hc_post to each workgroup's output rows; otherwise the layer and the
hc_post kernel. Either way the layer output and the post streams must equal,
bit for bit, those of xl_layer_forward_async followed by xl_hc_post_async, and
the post streams must equal the oracle's hc_post of that layer output
(oracle/xl_oracle.c orc_hc_post, pinned to sycl/hc/core.hpp:81-86).
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.test_gpu_parity import dev, kind_types, route, step

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

E = 24
# (dim, ff, k, H, one launch): the streaming kernel runs 4096 x 3072 and
# 5120 x 2304 up to 6 picks, 1024 x 512 and 256 x 768 up to 16
SHAPES = [(4096, 3072, 6, 4, True), (4096, 3072, 1, 1, True), (1024, 512, 16, 2, True), (256, 768, 12, 3, True),
          (5120, 2304, 6, 4, True), (4096, 3072, 8, 4, False)]


def bits(t):
    return t.cpu().numpy().view(np.uint32)


def both(lane, ids, w, x, res, post, comb, shared=None, in_place=False):
    """(out, post streams) of the one call and of the two calls, on one stream."""
    dim = x.shape[-1]
    H = res.shape[0]
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        y1 = torch.full((dim,), float("nan"), dtype=torch.float32, device="cuda")
        y2 = y1.clone()
        r1 = res.clone()
        p1 = r1 if in_place else torch.full((H, dim), float("nan"), dtype=torch.float32, device="cuda")
        p2 = torch.full((1, H, dim), float("nan"), dtype=torch.float32, device="cuda")
        lane.layer_forward_post_async(0, ids, w, x, y1, r1, post, comb, p1, shared=shared, stream=s.cuda_stream)
        lane.layer_forward_async(0, ids, w, x, y2, shared=shared, stream=s.cuda_stream)
        lane.hc_post_async(y2.view(1, dim), res.view(1, H, dim), post.view(1, 8), comb.view(1, 64), p2,
                           stream=s.cuda_stream)
    lane.sync(s.cuda_stream)
    torch.cuda.synchronize()
    return y1, p1, y2, p2.view(H, dim)


@pytest.mark.parametrize("kind", ["iq2", "iq1", "mixed"])
@pytest.mark.parametrize("dim,ff,k,H,fused", SHAPES)
def test_post_layer_matches_layer_then_post(orc, kind, dim, ff, k, H, fused):
    step(f"layer + hc_post {kind} dim={dim} ff={ff} k={k} H={H}")
    rng = np.random.default_rng(dim * 5 + ff + k + H)
    lane = xl.Lane(dim, ff, 1, E, kind_types(kind, E), max_picks=16)
    try:
        lane.generate(seed=61)
        for trial in range(3):
            ids, w = route(rng.standard_normal(E).astype(np.float32), k)
            x = rng.standard_normal(dim).astype(np.float32)
            res = rng.standard_normal((H, dim)).astype(np.float32)
            post = (rng.random(8) * 2).astype(np.float32)
            comb = rng.random(64).astype(np.float32)
            shared = rng.standard_normal(dim).astype(np.float32) if trial != 1 else None
            y1, p1, y2, p2 = both(lane, dev(ids), dev(w), dev(x), dev(res), dev(post), dev(comb),
                                  None if shared is None else dev(shared), in_place=trial == 2)
            assert np.array_equal(bits(y1), bits(y2)), trial
            assert np.array_equal(bits(p1), bits(p2)), trial
            want = orc.hc_post(y2.cpu().numpy().reshape(1, dim), res.reshape(1, H, dim), post.reshape(1, 8),
                               comb.reshape(1, 64), dim, H, 1)[0]
            assert np.array_equal(bits(p1), want.view(np.uint32)), trial
            assert np.all(np.isfinite(y1.cpu().numpy()))
            # the fused call applied hc_post inside its one launch (not the two-call fallback)
            assert lane.launch_counts()["post"] == (trial + 1 if fused else 0)
    finally:
        lane.close()


def test_post_layer_rejects_overlap(orc):
    step("layer + hc_post: overlapping output")
    lane = xl.Lane(1024, 512, 1, E, kind_types("iq2", E), max_picks=8)
    try:
        lane.generate(seed=61)
        ids, w = route(np.random.default_rng(3).standard_normal(E).astype(np.float32), 4)
        x = dev(np.ones(1024, np.float32))
        post, comb = dev(np.ones(8, np.float32)), dev(np.ones(64, np.float32))
        buf = torch.zeros(4 * 1024 + 1024, dtype=torch.float32, device="cuda")
        res = buf[:2 * 1024].view(2, 1024)
        out = torch.zeros(1024, dtype=torch.float32, device="cuda")
        with pytest.raises(xl.XLError, match="overlaps"):   # post streams half over the residual streams
            lane.layer_forward_post_async(0, dev(ids), dev(w), x, out, res, post, comb, buf[1024:3 * 1024].view(2, 1024))
        with pytest.raises(xl.XLError, match="overlaps"):   # post streams over the layer output
            lane.layer_forward_post_async(0, dev(ids), dev(w), x, buf[4 * 1024:], res, post, comb,
                                          buf[3 * 1024:5 * 1024].view(2, 1024))
        with pytest.raises(xl.XLError, match="overlaps"):   # layer output over the residual streams
            lane.layer_forward_post_async(0, dev(ids), dev(w), x, buf[1024:2048], res, post, comb,
                                          buf[3 * 1024:5 * 1024].view(2, 1024))
        assert lane.launch_counts()["post"] == 0
    finally:
        lane.close()
