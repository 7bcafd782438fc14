"""The no-allocation entry point (xl_shared_forward_noalloc) against the
workspace entry point it varies (xl_shared_forward_async), through the C ABI:
the same kernels on the same inputs, so the outputs must be bit-identical, on
two calls in a row (the second with fewer tokens, so it runs over what the
first left in the shared static scratch), and a token count whose
intermediates exceed the scratch is rejected."""
from __future__ import annotations

import sys

import numpy as np
import pytest

import crosslane_amd as xl
from tests.dense import dense_matrix

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def step(msg):
    print(f"[gpu-step] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


@pytest.mark.parametrize("types,ff,lim", [((13, 13, 14), 3072, 0.0), ((12, 12, 8), 2048, 7.0)])
def test_noalloc_matches_workspace_entry(types, ff, lim):
    dim = 4096
    t = np.zeros((1, 1, 3), np.int32)
    t[..., :2], t[..., 2] = 16, 17
    lane = xl.Lane(dim, 3072, 1, 1, t, max_picks=1, swiglu_limit=lim)
    try:
        mats = [dev(dense_matrix(types[0], ff, dim, ff)), dev(dense_matrix(types[1], ff, dim, ff + 1)),
                dev(dense_matrix(types[2], dim, ff, ff + 2))]
        for T in (5, 2):   # the second call is smaller and follows the first
            step(f"no-alloc shared FFN types={types} ff={ff} T={T} lim={lim}")
            x = dev((np.random.default_rng(ff + T).standard_normal((T, dim)) * 2.0).astype(np.float32))
            work = torch.empty(xl.shared_work_bytes(dim, ff, T), dtype=torch.uint8, device="cuda")
            want = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
            got = torch.full((T, dim), float("nan"), dtype=torch.float32, device="cuda")
            torch.cuda.synchronize()
            lane.shared_forward_async(types, *mats, ff, x, want, work)
            lane.shared_forward_noalloc(types, *mats, ff, x, got)
            lane.sync()
            assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32)), T
        # intermediates beyond the static scratch: a clear error, nothing launched
        T = 4096
        assert xl.shared_work_bytes(dim, ff, T) > 8 << 20
        x = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        out = torch.zeros((T, dim), dtype=torch.float32, device="cuda")
        with pytest.raises(xl.XLError, match="static scratch"):
            lane.shared_forward_noalloc(types, *mats, ff, x, out)
    finally:
        lane.close()
