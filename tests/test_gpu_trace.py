"""Bit-exact parity of the kernels that run the path, on their own data.

The north star's exact bars (Q8_K activation bytes and per-block int32
partials) are checked here on what the hot kernels themselves stage and form,
through the parity trace (xl_layer_trace_async, xl_grouped_trace_async): the
streaming kernel with its IQ2, IQ1_M and mixed-type instances (configs 0 to
3), the all-types kernel with its IQ2, IQ1_M and mixed-type instances, and the
grouped MFMA kernels
(config 4). For each launch:

* Q8_K(x) as staged: the 292-byte blocks equal the oracle's quant_block of x
  (q8k_core.hpp:30-38), bsums included;
* Q8_K(h) as staged: equal to the oracle's quant_block of the launch's own h
  (the SwiGLU's exp differs by ulps between host and device, so h itself is
  compared within tolerance; the reference's probe compares the same way,
  parity/hip_resident_check.cpp:91-127, warm/expert_check.cpp:86-88);
* every row's integer per 256-weight block, gate and up against Q8_K(x), down
  against Q8_K(h): equal to the oracle's block partials (the sum over the eight
  AVX2 lanes of integer_lane, q8k_core.hpp:43-69; IQ1_M as 8 * main + delta);
* the combined output within max relative error 1e-3 of the oracle chain.
"""
from __future__ import annotations

import numpy as np
import pytest

import crosslane_amd as xl
from oracle.oracle import Q8K_DTYPE
from tests.conftest import max_rel
from tests.test_gpu_grouped import token_routes
from tests.test_gpu_parity import TOL, dev, route, step, types_map

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 0x7A3CE


def zeros(n, dtype):
    return torch.zeros(n, dtype=dtype, device="cuda")


def check_pick(orc, sig, mats, dim, ff, q8x, h, q8h, ints, tag):
    """One pick's trace against the oracle: Q8_K(h) of the device's own h and the
    block integers of all its rows."""
    nbx, nbh = dim // 256, ff // 256
    want_q8h = orc.quantize(h)
    assert np.array_equal(q8h, want_q8h.view(np.uint8)), f"{tag}: Q8_K(h) bytes"
    gi = ints[:ff * nbx].reshape(ff, nbx)
    ui = ints[ff * nbx:2 * ff * nbx].reshape(ff, nbx)
    di = ints[2 * ff * nbx:].reshape(dim, nbh)
    assert np.array_equal(gi, orc.matrix_ints(sig[0], mats[0], ff, dim, q8x)), f"{tag}: gate block integers"
    assert np.array_equal(ui, orc.matrix_ints(sig[1], mats[1], ff, dim, q8x)), f"{tag}: up block integers"
    assert np.array_equal(di, orc.matrix_ints(sig[2], mats[2], dim, ff, want_q8h)), f"{tag}: down block integers"


LAYER_CASES = [
    # (XL_LAYER_PATH, dim, ff, E, k, layer type map kind, expected kernel)
    ("1", 4096, 3072, 12, 6, "iq2", 1),     # config 1: the streaming kernel
    ("1", 4096, 3072, 12, 1, "iq2", 1),     # config 0: one pick (1-2 pick instance)
    ("4", 4096, 3072, 12, 3, "iq2", 1),     # 3-4 pick instance
    ("1", 1024, 512, 8, 6, "iq2", 1),
    ("1", 4096, 3072, 12, 6, "iq1", 1),     # config 2: the streaming kernel's IQ1_M instance
    ("1", 4096, 3072, 12, 6, "mixed", 1),   # config 3: its mixed instance (descriptors)
    ("4", 4096, 3072, 12, 1, "iq1", 1),
    ("4", 4096, 3072, 12, 3, "mixed", 1),
    ("4", 1024, 512, 8, 8, "mixed", 1),
    ("4", 256, 768, 6, 5, "iq1", 1),
    ("3", 4096, 3072, 12, 6, "iq2", 3),     # all-types kernel, IQ2 instance
    ("3", 4096, 3072, 12, 6, "iq1", 3),     # IQ1_M-only instance
    ("3", 4096, 3072, 12, 6, "mixed", 3),   # mixed types, descriptors
    ("3", 1024, 512, 8, 5, "mixed", 3),
    ("3", 256, 768, 6, 4, "iq1", 3),
]


def layer_types(kind, E):
    if kind == "iq2":
        return types_map(1, E, 16, 17)
    if kind == "iq1":
        return types_map(1, E, 29, 29)
    rng = np.random.default_rng(E)
    t = rng.choice([16, 17, 29], size=E)
    t[:3] = [16, 17, 29]   # every type present
    return np.repeat(t.reshape(1, E, 1), 3, axis=-1).astype(np.int32)


@pytest.mark.parametrize("path,dim,ff,E,k,kind,kernel", LAYER_CASES)
def test_layer_trace_bit_exact(orc, monkeypatch, path, dim, ff, E, k, kind, kernel):
    monkeypatch.setenv("XL_LAYER_PATH", path)
    step(f"layer trace path={path} dim={dim} ff={ff} E={E} k={k} {kind}")
    types = layer_types(kind, E)
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=8)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(dim + ff + k)
        ids, w = route(rng.standard_normal(E).astype(np.float32), k)
        x = rng.standard_normal(dim).astype(np.float32)
        nbx, nbh = dim // 256, ff // 256
        rec = 2 * ff * nbx + dim * nbh
        out = zeros(dim, torch.float32)
        q8x = zeros(nbx * 292, torch.uint8)
        q8h = zeros(k * nbh * 292, torch.uint8)
        h = zeros(k * ff, torch.float32)
        ints = zeros(k * rec, torch.int32)
        torch.cuda.synchronize()
        ran = lane.layer_trace_async(0, dev(ids), dev(w), dev(x), out, q8x, q8h, h, ints)
        lane.sync()
        assert ran == kernel
        want_q8x = orc.quantize(x)
        assert np.array_equal(q8x.cpu().numpy(), want_q8x.view(np.uint8)), "Q8_K(x) bytes"
        h, q8h, ints = h.cpu().numpy().reshape(k, ff), q8h.cpu().numpy().reshape(k, -1), ints.cpu().numpy().reshape(k, rec)
        rows = []
        for i, e in enumerate(ids):
            sig = tuple(int(v) for v in types[0, e])
            mats = orc.gen_expert(sig, SEED, 0, int(e), dim, ff)
            check_pick(orc, sig, mats, dim, ff, want_q8x, h[i], q8h[i], ints[i], f"pick {i} (expert {e}, {sig})")
            rows.append(orc.expert(sig, *mats, dim, ff, x))
        assert max_rel(out.cpu().numpy(), orc.combine(ids, w, np.stack(rows))) < TOL
        # the traced launch computes what the untraced one does
        plain = lane.layer_forward(0, ids, w, x)
        assert np.array_equal(plain.view(np.uint32), out.cpu().numpy().view(np.uint32))
    finally:
        lane.close()


@pytest.mark.parametrize("dim,ff,E,T,k,skewed", [(1024, 512, 8, 40, 8, True), (4096, 3072, 24, 24, 6, False)])
def test_grouped_trace_bit_exact(orc, monkeypatch, dim, ff, E, T, k, skewed):
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    step(f"grouped trace dim={dim} ff={ff} E={E} T={T} k={k} skewed={skewed}")
    types = types_map(1, E, 16, 17)
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=8, max_tokens=64)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(dim + T)
        skew = np.where(np.arange(E) < 3, 4.0, 0.0).astype(np.float32) if skewed else None
        ids, w = token_routes(rng, T, E, k, skew)
        x = rng.standard_normal((T, dim)).astype(np.float32)
        nbx, nbh, P = dim // 256, ff // 256, T * k
        rec = 2 * ff * nbx + dim * nbh
        out = zeros((T, dim), torch.float32)
        q8x = zeros(T * nbx * 292, torch.uint8)
        q8h = zeros(P * nbh * 292, torch.uint8)
        h = zeros(P * ff, torch.float32)
        ints = zeros(P * rec, torch.int32)
        torch.cuda.synchronize()
        lane.grouped_trace_async(0, dev(ids), dev(w), dev(x), out, q8x, q8h, h, ints)
        lane.sync()
        q8x = q8x.cpu().numpy().reshape(T, -1)
        h, q8h, ints = h.cpu().numpy().reshape(P, ff), q8h.cpu().numpy().reshape(P, -1), ints.cpu().numpy().reshape(P, rec)
        cache = {}
        for t in range(T):
            want_q8x = orc.quantize(x[t])
            assert np.array_equal(q8x[t], want_q8x.view(np.uint8)), f"token {t}: Q8_K(x) bytes"
            # every pair of a few tokens in full, the rest of the pairs by their Q8_K(h) bytes
            for i, e in enumerate(ids[t]):
                p = t * k + i
                if t < 3:
                    if int(e) not in cache:
                        cache[int(e)] = orc.gen_expert((16, 16, 17), SEED, 0, int(e), dim, ff)
                    check_pick(orc, (16, 16, 17), cache[int(e)], dim, ff, want_q8x, h[p], q8h[p], ints[p],
                               f"token {t} pick {i} (expert {e})")
                else:
                    assert np.array_equal(q8h[p], orc.quantize(h[p]).view(np.uint8)), f"pair {p}: Q8_K(h) bytes"
        plain = lane.grouped_forward(0, ids, w, x)
        assert np.array_equal(plain.view(np.uint32), out.cpu().numpy().view(np.uint32))
    finally:
        lane.close()


def test_trace_rejects_separate_launch_layers(monkeypatch):
    monkeypatch.setenv("XL_LAYER_PATH", "0")   # separate launches: no single launch to trace
    lane = xl.Lane(1024, 512, 1, 4, types_map(1, 4, 16, 17), max_picks=4)
    try:
        lane.generate(SEED)
        ids = dev(np.array([0, 1], np.int32)); w = dev(np.array([0.5, 0.5], np.float32))
        x = dev(np.zeros(1024, np.float32)); out = zeros(1024, torch.float32)
        with pytest.raises(xl.XLError, match="single launch"):
            lane.layer_trace_async(0, ids, w, x, out, q8x=zeros(4 * 292, torch.uint8))
    finally:
        lane.close()
