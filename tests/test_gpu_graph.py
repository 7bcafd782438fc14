"""Layer calls captured in a HIP graph and replayed.

The streaming kernel takes its h-exchange parity from a device counter that
the last workgroup of each launch advances, never from the host, so a captured
launch replayed many times must alternate the exchange buffers as eager
launches do. Each replay runs on new inputs copied into the captured buffers;
eager calls and synchronizations run between the replays, and every replay's
output must equal the eager call's on the same inputs bit for bit (and stay
within 1e-3 of the oracle). The capture stream is also the eager calls' stream,
so the context's cross-stream ordering adds no wait on an event outside the
capture.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.test_gpu_parity import TOL, dev, kind_types, route, step

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 0x6A7


@pytest.mark.parametrize("kind,dim,ff,k", [("iq2", 4096, 3072, 6), ("iq1", 4096, 3072, 6), ("mixed", 4096, 3072, 4),
                                           ("iq2", 5120, 2304, 6), ("iq2", 4096, 3072, 1)])
def test_captured_layer_replays(orc, kind, dim, ff, k):
    step(f"graph capture: {kind} {dim}x{ff} k={k}")
    E = 16
    types = kind_types(kind, E)
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=8)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(dim + k)
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            g_ids = torch.zeros(k, dtype=torch.int32, device="cuda")
            g_w = torch.zeros(k, dtype=torch.float32, device="cuda")
            g_x = torch.zeros(dim, dtype=torch.float32, device="cuda")
            g_out = torch.zeros(dim, dtype=torch.float32, device="cuda")
            e_out = torch.zeros(dim, dtype=torch.float32, device="cuda")

        def inputs():
            ids, w = route(rng.standard_normal(E).astype(np.float32), k)
            return ids, w, rng.standard_normal(dim).astype(np.float32)

        ids, w, x = inputs()
        with torch.cuda.stream(s):
            g_ids.copy_(dev(ids)); g_w.copy_(dev(w)); g_x.copy_(dev(x))
            for _ in range(3):   # eager calls on the capture stream first
                lane.layer_forward_async(0, g_ids, g_w, g_x, e_out, stream=s.cuda_stream)
        s.synchronize()
        lane.sync(s.cuda_stream)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            lane.layer_forward_async(0, g_ids, g_w, g_x, g_out, stream=s.cuda_stream)
        before = lane.launch_counts()
        for rep in range(6):
            ids, w, x = inputs()
            with torch.cuda.stream(s):
                g_ids.copy_(dev(ids)); g_w.copy_(dev(w)); g_x.copy_(dev(x))
                graph.replay()
                # the same inputs eagerly, on the same stream, after the replay
                lane.layer_forward_async(0, g_ids, g_w, g_x, e_out, stream=s.cuda_stream)
            s.synchronize()
            lane.sync(s.cuda_stream)
            got, want = g_out.cpu().numpy(), e_out.cpu().numpy()
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (rep, max_rel(got, want))
            rows = []
            for e in ids:
                sig = tuple(int(v) for v in types[0, e])
                rows.append(orc.expert(sig, *orc.gen_expert(sig, SEED, 0, int(e), dim, ff), dim, ff, x))
            assert max_rel(got, orc.combine(ids, w, np.stack(rows))) < TOL, rep
        # the eager calls ran the streaming kernel (the replays do not pass through the library)
        assert lane.launch_counts()["stream"] - before["stream"] == 6
    finally:
        lane.close()
