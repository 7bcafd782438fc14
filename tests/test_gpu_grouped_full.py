"""The grouped path at benchmark config 4's full size: 512 tokens, each routed
top-6 over 384 experts (d_model 4096, d_ff 3072, IQ2_XXS gate/up + IQ2_XS
down), a max_tokens = 512 workspace, thousands of (token, pick) pairs bucketed
into hundreds of 16-pair tasks. The MFMA kernels are forced
(XL_GROUPED_PATH=2). Bars: every token within max relative error 1e-3 of a
per-token layer call on the device, a sample of tokens within 1e-3 of the
oracle, and a rerun bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.test_gpu_grouped import token_routes
from tests.test_gpu_parity import TOL, dev, step, types_map

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

DIM, FF, E, T, K, SEED = 4096, 3072, 384, 512, 6, 0x4C4


def test_grouped_config4_full(orc, monkeypatch):
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    step(f"grouped full: T={T} E={E} k={K} dim={DIM} ff={FF} max_tokens={T}")
    lane = xl.Lane(DIM, FF, 1, E, types_map(1, E, 16, 17), max_picks=8, max_tokens=T)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(SEED)
        ids, w = token_routes(rng, T, E, K)
        x = rng.standard_normal((T, DIM)).astype(np.float32)
        d_ids, d_w, d_x = dev(ids), dev(w), dev(x)
        out = torch.zeros((T, DIM), dtype=torch.float32, device="cuda")
        again = torch.zeros_like(out)
        per = torch.zeros_like(out)
        torch.cuda.synchronize()   # the fills above ran on torch's stream, the lane runs on its own
        lane.grouped_forward_async(0, d_ids, d_w, d_x, out)
        lane.grouped_forward_async(0, d_ids, d_w, d_x, again)
        step("grouped full: per-token layer calls")
        for t in range(T):
            lane.layer_forward_async(0, d_ids[t], d_w[t], d_x[t], per[t])
        lane.sync()
        got, got2, want_dev = out.cpu().numpy(), again.cpu().numpy(), per.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), got2.view(np.uint32))
        worst = max(max_rel(got[t], want_dev[t]) for t in range(T))
        assert worst < TOL, worst
        step(f"grouped full: worst per-token max_rel vs layer calls {worst:.3e}; oracle sample")
        cache = {}
        for t in rng.choice(T, size=6, replace=False):
            rows = []
            for e in ids[t]:
                if int(e) not in cache:
                    cache[int(e)] = orc.gen_expert((16, 16, 17), SEED, 0, int(e), DIM, FF)
                rows.append(orc.expert((16, 16, 17), *cache[int(e)], DIM, FF, x[t]))
            want = orc.combine(ids[t], w[t], np.stack(rows))
            assert max_rel(got[t], want) < TOL, (int(t), max_rel(got[t], want))
    finally:
        lane.close()
