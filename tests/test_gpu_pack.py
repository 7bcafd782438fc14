"""GPU: a weight pack in the reference's layout loads losslessly (every matrix
downloads to the pack's own bytes) and the layer computes from it what the
oracle computes from the pack's bytes."""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.packs import write_pack
from tests.test_gpu_parity import TOL, step

pytestmark = pytest.mark.gpu


def test_pack_load_roundtrip_and_layer(orc, tmp_path):
    dim, ff, E = 1024, 512, 6
    sigs = [(16, 16, 16), (16, 16, 17), (29, 29, 29), (17, 17, 29)]
    step("pack load")
    p = write_pack(str(tmp_path / "pack"), orc, sigs, dim, ff, E, seed=9)
    first, L = 1, 3
    types = xl.pack_types(p, first, L, E)
    lane = xl.Lane(dim, ff, L, E, types, max_picks=4)
    try:
        lane.load_pack(p, first_layer=first)
        for l in range(L):
            for e in range(E):
                for r in range(3):
                    n, k = (ff, dim) if r < 2 else (dim, ff)
                    want = orc.gen_matrix(int(types[l, e, r]), 9, first + l, e, r, n, k)
                    assert np.array_equal(lane.download(l, e, r), want), (l, e, r)
        rng = np.random.default_rng(4)
        for l in range(L):
            ids = rng.permutation(E)[:4].astype(np.int32)
            w = rng.random(4).astype(np.float32)
            x = rng.standard_normal(dim).astype(np.float32)
            tt = tuple(int(v) for v in types[l, 0])
            rows = [orc.expert(tt, *orc.gen_expert(tt, 9, first + l, int(e), dim, ff), dim, ff, x) for e in ids]
            want = orc.combine(ids, w, np.stack(rows))
            got = lane.layer_forward(l, ids, w, x)
            assert max_rel(got, want) < TOL, (l, max_rel(got, want))
        with pytest.raises(xl.XLError, match="layer window"):
            lane.load_pack(p, first_layer=2)
    finally:
        lane.close()
