"""GPU parity of the MoE block call (xl_moe_block_async): the routed layer of
one token, the shared-expert FFN added last and the hyper-connection post of
the sum (hip_backend.cpp:635-711 with the shared expert of :664-666, then :777
k4::hc_post). The block's output and post streams must equal, bit for bit,
those of xl_shared_forward_async into a shared row followed by
xl_layer_forward_post_async with that row: the shared FFN's x quantization
moves into the streaming launch and the final sum and hc_post into the shared
down rows' epilogue, but every value is the same operation on the same
operands. With a layer the streaming kernel does not run (4096 x 3072 at eight
picks) the block takes its separate-launch route, with the same bits. The
block captured in a HIP graph replays on new inputs with the eager call's bits.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.dense import dense_matrix
from tests.test_gpu_parity import dev, kind_types, route, step

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

E = 24
# (dim, ff, shared ff, shared types, k, H, one streaming launch)
SHAPES = [(4096, 3072, 3072, (13, 13, 14), 6, 4, True), (4096, 3072, 2048, (12, 12, 8), 1, 1, True),
          (1024, 512, 768, (14, 14, 13), 16, 2, True), (5120, 2304, 1024, (13, 13, 14), 6, 4, True),
          (4096, 3072, 1024, (13, 13, 14), 8, 3, False)]


def bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("kind", ["iq2", "iq1", "mixed"])
@pytest.mark.parametrize("dim,ff,sff,st,k,H,fused", SHAPES)
def test_moe_block_matches_shared_then_post_layer(kind, dim, ff, sff, st, k, H, fused):
    step(f"MoE block {kind} dim={dim} ff={ff} shared ff={sff} types={st} k={k} H={H}")
    rng = np.random.default_rng(dim + ff + sff + k + H)
    lane = xl.Lane(dim, ff, 1, E, kind_types(kind, E), max_picks=16, swiglu_limit=7.0 if k == 6 else 0.0)
    try:
        lane.generate(seed=71)
        g = dev(dense_matrix(st[0], sff, dim, 72))
        u = dev(dense_matrix(st[1], sff, dim, 73))
        dn = dev(dense_matrix(st[2], dim, sff, 74))
        work = torch.empty(xl.shared_work_bytes(dim, sff, 1), dtype=torch.uint8, device="cuda")
        work2 = torch.empty_like(work)
        s = torch.cuda.Stream()
        for trial in range(3):
            ids, w = route(rng.standard_normal(E).astype(np.float32), k)
            x = dev((rng.standard_normal(dim) * 2.0).astype(np.float32))
            res = dev(rng.standard_normal((H, dim)).astype(np.float32))
            post = dev((rng.random(8) * 2).astype(np.float32))
            comb = dev(rng.random(64).astype(np.float32))
            d_ids, d_w = dev(ids), dev(w)
            with torch.cuda.stream(s):
                y1 = torch.full((dim,), float("nan"), dtype=torch.float32, device="cuda")
                y2, sh = y1.clone(), y1.clone()
                r1 = res.clone()
                p1 = r1 if trial == 2 else torch.full((H, dim), float("nan"), dtype=torch.float32, device="cuda")
                p2 = torch.full((H, dim), float("nan"), dtype=torch.float32, device="cuda")
                lane.moe_block_async(0, d_ids, d_w, x, st, g, u, dn, sff, work, r1, post, comb, y1, p1,
                                     stream=s.cuda_stream)
                lane.shared_forward_async(st, g, u, dn, sff, x.view(1, dim), sh.view(1, dim), work2,
                                          stream=s.cuda_stream)
                lane.layer_forward_post_async(0, d_ids, d_w, x, y2, res, post, comb, p2, shared=sh,
                                              stream=s.cuda_stream)
            lane.sync(s.cuda_stream)
            torch.cuda.synchronize()
            assert np.array_equal(bits(y1), bits(y2)), trial
            assert np.array_equal(bits(p1), bits(p2)), trial
            assert np.all(np.isfinite(y1.cpu().numpy()))
            # the streaming launch quantized x for the shared FFN (not a quant32 launch)
            assert lane.launch_counts()["block"] == (trial + 1 if fused else 0)
    finally:
        lane.close()


def test_moe_block_rejects_bad_arguments():
    step("MoE block: overlaps and a short workspace")
    dim, sff, st, H = 1024, 768, (13, 13, 14), 2
    lane = xl.Lane(dim, 512, 1, E, kind_types("iq2", E), max_picks=8)
    try:
        lane.generate(seed=71)
        g, u = dev(dense_matrix(st[0], sff, dim, 72)), dev(dense_matrix(st[1], sff, dim, 73))
        dn = dev(dense_matrix(st[2], dim, sff, 74))
        ids, w = route(np.random.default_rng(3).standard_normal(E).astype(np.float32), 4)
        d_ids, d_w = dev(ids), dev(w)
        post, comb = dev(np.ones(8, np.float32)), dev(np.ones(64, np.float32))
        work = torch.empty(xl.shared_work_bytes(dim, sff, 1), dtype=torch.uint8, device="cuda")
        x = dev(np.ones(dim, np.float32))
        res = torch.zeros((H, dim), dtype=torch.float32, device="cuda")
        out = torch.zeros(dim, dtype=torch.float32, device="cuda")
        p = torch.zeros((H, dim), dtype=torch.float32, device="cuda")
        with pytest.raises(xl.XLError, match="workspace smaller"):
            lane.moe_block_async(0, d_ids, d_w, x, st, g, u, dn, sff, work[:1024], res, post, comb, out, p)
        with pytest.raises(xl.XLError, match="block output overlaps"):   # out over x
            lane.moe_block_async(0, d_ids, d_w, x, st, g, u, dn, sff, work, res, post, comb, x, p)
        with pytest.raises(xl.XLError, match="overlap"):                 # post streams over out
            buf = torch.zeros(3 * dim, dtype=torch.float32, device="cuda")
            lane.moe_block_async(0, d_ids, d_w, x, st, g, u, dn, sff, work, res, post, comb, buf[:dim],
                                 buf[dim // 2:dim // 2 + H * dim].view(H, dim))
        assert lane.launch_counts()["block"] == 0
    finally:
        lane.close()


def test_moe_block_captured_in_a_graph_replays():
    """The block's four launches captured in a HIP graph: each replay on new
    inputs (copied into the captured buffers) equals the eager call on the same
    inputs bit for bit, with eager calls and synchronizations between replays."""
    dim, ff, sff, st, k, H = 4096, 3072, 3072, (13, 13, 14), 6, 4
    step("MoE block: graph capture and replays")
    rng = np.random.default_rng(77)
    lane = xl.Lane(dim, ff, 1, E, kind_types("iq2", E), max_picks=8)
    try:
        lane.generate(seed=71)
        g = dev(dense_matrix(st[0], sff, dim, 72))
        u = dev(dense_matrix(st[1], sff, dim, 73))
        dn = dev(dense_matrix(st[2], dim, sff, 74))
        work = torch.empty(xl.shared_work_bytes(dim, sff, 1), dtype=torch.uint8, device="cuda")
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            c_ids = torch.zeros(k, dtype=torch.int32, device="cuda")
            c_w = torch.zeros(k, dtype=torch.float32, device="cuda")
            c_x = torch.zeros(dim, dtype=torch.float32, device="cuda")
            c_res = torch.zeros((H, dim), dtype=torch.float32, device="cuda")
            c_post = torch.zeros(8, dtype=torch.float32, device="cuda")
            c_comb = torch.zeros(64, dtype=torch.float32, device="cuda")
            g_out, e_out = torch.zeros(dim, device="cuda"), torch.zeros(dim, device="cuda")
            g_p, e_p = torch.zeros((H, dim), device="cuda"), torch.zeros((H, dim), device="cuda")

        def load_inputs():
            ids, w = route(rng.standard_normal(E).astype(np.float32), k)
            with torch.cuda.stream(s):
                c_ids.copy_(dev(ids)); c_w.copy_(dev(w))
                c_x.copy_(dev((rng.standard_normal(dim) * 2.0).astype(np.float32)))
                c_res.copy_(dev(rng.standard_normal((H, dim)).astype(np.float32)))
                c_post.copy_(dev((rng.random(8) * 2).astype(np.float32)))
                c_comb.copy_(dev(rng.random(64).astype(np.float32)))

        def block(out, p):
            lane.moe_block_async(0, c_ids, c_w, c_x, st, g, u, dn, sff, work, c_res, c_post, c_comb, out, p,
                                 stream=s.cuda_stream)

        load_inputs()
        with torch.cuda.stream(s):
            for _ in range(3):   # eager calls on the capture stream first
                block(e_out, e_p)
        s.synchronize()
        lane.sync(s.cuda_stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            block(g_out, g_p)
        for rep in range(5):
            load_inputs()
            with torch.cuda.stream(s):
                graph.replay()
                block(e_out, e_p)   # the same inputs eagerly, after the replay
            s.synchronize()
            lane.sync(s.cuda_stream)
            assert np.array_equal(bits(g_out), bits(e_out)), rep
            assert np.array_equal(bits(g_p), bits(e_p)), rep
            assert np.all(np.isfinite(g_out.cpu().numpy()))
    finally:
        lane.close()
