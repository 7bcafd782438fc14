"""The reference's Q8_K edge blocks through every kernel that computes the path.

x is built from the 13 golden blocks written from the reference's own
quant_block (q8k_core.hpp:25-38; tests/golden: an all-zero block, .5 ties, an
equal-magnitude tie of opposite signs, one-hot blocks, a subnormal largest
magnitude, a 2.5e30 block), two crafted blocks whose largest magnitude sits
just below and just above 127 / FLT_MAX (is = -127/mx overflows to -inf in the
first, d = 1/is = -0), and one N(0,1) block. It is run through the parity
trace of the streaming kernel (IQ2, IQ1_M and mixed-type instances, one to
six picks, at 4096 x 3072 and at 5120 x 2304, where x takes four more blocks
of the other set), the all-types kernel and the grouped MFMA kernels (token
rows), and the staged Q8_K(x) must equal the golden bytes (and the oracle's,
for the crafted blocks) byte for byte: the bar the reference's probe applies
to its working lane's own .q8k bytes (parity/hip_resident_check.cpp:91-127).

The SwiGLU limit 7 (the model's own clamp, q8k_core.hpp:92-95) keeps h finite
when a 2.5e30 block drives the gate rows to ~1e29; Q8_K(h) and every row's
block integers are then checked as in test_gpu_trace.py.

The float results are held to a float64 evaluation of the same exact block
integers (h from the gate/up integers and scales; the output from the down
integers and the launch's own Q8_K(h) scales), within 1e-3, not to the oracle
chain: on this input the reference's float order (eight lane chains, IQ1_M's
main and delta sums apart, q8k_core.hpp:76-91) cancels catastrophically where
a row's terms of the 2.5e30 block nearly cancel (one seed's gate row comes out
of the oracle with the wrong sign and ~1e28 too large), so the oracle itself is
not within 1e-3 of the exact value there. The kernels form each block's
integer exactly and scale it once, and stay within the bar.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import max_rel
from tests.test_gpu_parity import TOL, dev, route, step
from tests.test_gpu_trace import check_pick, layer_types, zeros

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

SEED = 0x0E09E
LIM = 7.0
DIM, FF, E = 4096, 3072, 12


def edge_x(shift: int = 0):
    """(x, expected Q8_K bytes per block): 16 blocks, the golden ones first
    (rotated by `shift` blocks), bytes from the golden file where it has them."""
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))
    gx, gb = gold["q8k_x"], gold["q8k_bytes"]
    rng = np.random.default_rng(99)
    tiny = (rng.standard_normal(256) * 1e-39).astype(np.float32)
    tiny[17] = 1.0e-38                      # largest magnitude, positive: is = -inf, d = -0
    edge = (rng.standard_normal(256) * 1e-38).astype(np.float32)
    edge[200] = -4.0e-37                    # just above 127 / FLT_MAX: is finite, huge
    blocks = list(gx) + [tiny, edge, rng.standard_normal(256).astype(np.float32)]
    want = list(gb) + [None, None, None]
    order = [(i + shift) % 16 for i in range(16)]
    return np.concatenate([blocks[i] for i in order]).astype(np.float32), [want[i] for i in order]


def tie_x():
    """(x, None bytes): 16 crafted blocks whose largest magnitude M occurs more
    than once with both signs, in different lanes (4 values per lane) and within
    one lane, in either order; the first occurrence sets the sign of mx
    (q8k_core.hpp:33's strict '>' scan). Expected bytes come from the oracle."""
    rng = np.random.default_rng(7)
    cases = [((5, 1), (9, -1)), ((5, -1), (9, 1)), ((4, -1), (6, 1)), ((6, 1), (7, -1)), ((6, -1), (7, 1)),
             ((200, 1), (100, -1)), ((0, 1), (3, -1)), ((0, -1), (1, 1)), ((254, -1), (255, 1)),
             ((252, -1), (253, 1), (2, 1)), ((128, 1), (64, -1), (65, 1)), ((17, -1), (18, -1), (19, 1))]
    blocks = []
    for pos in cases:
        b = (rng.standard_normal(256) * 0.5).astype(np.float32)
        for i, sg in pos:
            b[i] = np.float32(3.0 * sg)
        blocks.append(b)
    alt = np.full(256, 2.0, np.float32) * np.where(np.arange(256) % 2, 1, -1).astype(np.float32)
    blocks.append(alt)                                         # every value a tie, the first negative
    blocks.append(np.where(np.arange(256) % 3 == 0, -0.0, 0.0).astype(np.float32))   # zero block with -0
    one = np.zeros(256, np.float32); one[255] = -1.5
    blocks.append(one)
    blocks.append(rng.standard_normal(256).astype(np.float32))
    return np.concatenate(blocks).astype(np.float32), [None] * 16


def x_for(dim, ties, shift):
    """(x, expected bytes per block) of dim values: the tie or edge blocks, then
    (dim above 4096) the first blocks of the other set."""
    x, want = tie_x() if ties else edge_x(shift=shift)
    extra = (dim - 4096) // 256
    if extra > 0:
        x2, want2 = edge_x(shift=shift) if ties else tie_x()
        x = np.concatenate([x, x2[:256 * extra]])
        want = list(want) + list(want2[:extra])
    return x.astype(np.float32), want


def block_scales(t, mat, rows):
    """fp16 block scales of an AoS matrix as float64 [rows, blocks] (IQ1_M: the
    scale split over the top nibbles of the four scale words)."""
    bb = {16: 66, 17: 74, 29: 56}[t]
    b = np.ascontiguousarray(mat).reshape(-1).view(np.uint8).reshape(rows, -1, bb)
    if t != 29:
        h = b[..., 0:2].copy().view("<u2")[..., 0]
    else:
        sc = b[..., 48:56].copy().view("<u2").astype(np.uint32)
        h = ((sc[..., 0] >> 12) | ((sc[..., 1] >> 8) & 0xF0) | ((sc[..., 2] >> 4) & 0xF00) | (sc[..., 3] & 0xF000))
        h = h.astype(np.uint16)
    return h.view(np.float16).astype(np.float64)


def exact_h(sig, mats, ints, q8x, dim=DIM, ff=FF):
    """h of one pick in float64 from the exact gate/up block integers."""
    DIM, FF = dim, ff
    nbx = DIM // 256
    dx = q8x["d"].astype(np.float64)
    gi = ints[:FF * nbx].reshape(FF, nbx).astype(np.float64)
    ui = ints[FF * nbx:2 * FF * nbx].reshape(FF, nbx).astype(np.float64)
    g = 0.125 * np.sum(block_scales(sig[0], mats[0], FF) * dx * gi, axis=1)
    u = 0.125 * np.sum(block_scales(sig[1], mats[1], FF) * dx * ui, axis=1)
    g = np.minimum(g, LIM)
    u = np.clip(u, -LIM, LIM)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-g)) * u


def exact_y(sig, mats, ints, q8h_bytes, dim=DIM, ff=FF):
    """One pick's output row in float64 from the exact down block integers and
    the launch's own Q8_K(h) scales."""
    DIM, FF = dim, ff
    nbx, nbh = DIM // 256, FF // 256
    dh = q8h_bytes.reshape(nbh, 292)[:, :4].copy().view(np.float32)[:, 0].astype(np.float64)
    di = ints[2 * FF * nbx:].reshape(DIM, nbh).astype(np.float64)
    return 0.125 * np.sum(block_scales(sig[2], mats[2], DIM) * dh * di, axis=1)


def check_exact(sig, mats, ints, q8x, h, q8h_bytes, tag, dim=DIM, ff=FF):
    h64 = exact_h(sig, mats, ints, q8x, dim, ff)
    assert max_rel(h, h64) < TOL, (tag, max_rel(h, h64))
    return exact_y(sig, mats, ints, q8h_bytes, dim, ff)


def check_q8x(orc, x, want_gold, q8x, tag):
    nb = x.size // 256
    want = orc.quantize(x).view(np.uint8).reshape(nb, 292)
    q8x = q8x.reshape(nb, 292)
    for b in range(nb):
        if want_gold[b] is not None:
            assert np.array_equal(want[b], want_gold[b]), f"{tag}: oracle vs golden, block {b}"
        assert np.array_equal(q8x[b], want[b]), f"{tag}: Q8_K(x) block {b}"
    return want.reshape(-1).view(orc.quantize(x).dtype)


def test_crafted_blocks_hit_the_overflow():
    # the crafted blocks' -127 / mx really overflows (first) and stays finite (second)
    x, _ = edge_x()
    with np.errstate(over="ignore"):
        assert np.isinf(np.float32(-127.0) / np.float32(1.0e-38))
        assert np.isfinite(np.float32(-127.0) / np.float32(-4.0e-37))
    assert np.max(np.abs(x[13 * 256:14 * 256])) == np.float32(1.0e-38)


LAYER_CASES = [
    # (XL_LAYER_PATH, layer type map kind, k, expected kernel, dim)
    ("4", "iq2", 6, 1, 4096),     # streaming kernel, IQ2 instance (config 1)
    ("4", "iq2", 1, 1, 4096),     # its one-pick instance (config 0)
    ("4", "iq1", 6, 1, 4096),     # IQ1_M instance (config 2)
    ("4", "mixed", 6, 1, 4096),   # mixed instance (config 3)
    ("3", "iq2", 6, 3, 4096),     # all-types kernel
    ("3", "iq1", 4, 3, 4096),
    ("3", "mixed", 6, 3, 4096),
    # 5120 x 2304 (config 6): 20-row bands, one down step up to six picks
    ("4", "iq2", 6, 1, 5120),     # config 6
    ("4", "iq2", 2, 1, 5120),
    ("4", "iq1", 6, 1, 5120),
    ("4", "mixed", 2, 1, 5120),
    ("4", "mixed", 6, 1, 5120),   # two steps, quantized as at 4096
]


@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("path,kind,k,kernel,dim", LAYER_CASES)
def test_layer_kernels_stage_golden_q8k(orc, monkeypatch, path, kind, k, kernel, dim, ties):
    monkeypatch.setenv("XL_LAYER_PATH", path)
    step(f"Q8_K edge blocks: layer path={path} {kind} k={k} dim={dim} ties={ties}")
    DIM, FF = dim, {4096: 3072, 5120: 2304}[dim]
    types = layer_types(kind, E)
    lane = xl.Lane(DIM, FF, 1, E, types, max_picks=8, swiglu_limit=LIM)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(k + len(kind))
        ids, w = route(rng.standard_normal(E).astype(np.float32), k)
        x, want_gold = x_for(DIM, ties, k)
        nbx, nbh = DIM // 256, FF // 256
        rec = 2 * FF * nbx + DIM * nbh
        out = zeros(DIM, torch.float32)
        q8x = zeros(nbx * 292, torch.uint8)
        q8h = zeros(k * nbh * 292, torch.uint8)
        h = zeros(k * FF, torch.float32)
        ints = zeros(k * rec, torch.int32)
        torch.cuda.synchronize()
        ran = lane.layer_trace_async(0, dev(ids), dev(w), dev(x), out, q8x, q8h, h, ints)
        lane.sync()
        assert ran == kernel
        want_q8x = check_q8x(orc, x, want_gold, q8x.cpu().numpy(), f"path {path} {kind} k={k}")
        h, q8h, ints = h.cpu().numpy().reshape(k, FF), q8h.cpu().numpy().reshape(k, -1), ints.cpu().numpy().reshape(k, rec)
        assert np.all(np.isfinite(h))
        y64 = np.zeros(DIM)
        for i, e in enumerate(ids):
            sig = tuple(int(v) for v in types[0, e])
            mats = orc.gen_expert(sig, SEED, 0, int(e), DIM, FF)
            tag = f"pick {i} (expert {e}, {sig})"
            check_pick(orc, sig, mats, DIM, FF, want_q8x, h[i], q8h[i], ints[i], tag)
            y64 += float(w[i]) * check_exact(sig, mats, ints[i], want_q8x, h[i], q8h[i], tag, DIM, FF)
        assert max_rel(out.cpu().numpy(), y64) < TOL
    finally:
        lane.close()


def test_grouped_kernels_stage_golden_q8k(orc, monkeypatch):
    monkeypatch.setenv("XL_GROUPED_PATH", "2")
    T, k = 4, 6
    step(f"Q8_K edge blocks: grouped T={T} k={k}")
    types = layer_types("iq2", E)
    lane = xl.Lane(DIM, FF, 1, E, types, max_picks=8, max_tokens=T, swiglu_limit=LIM)
    try:
        lane.generate(SEED)
        rng = np.random.default_rng(5)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
        w = (rng.random((T, k)) + 0.1).astype(np.float32)
        xs = [edge_x(shift=3 * t) for t in range(T)]
        x = np.stack([v for v, _ in xs])
        nbx, nbh, P = DIM // 256, FF // 256, T * k
        rec = 2 * FF * nbx + DIM * nbh
        out = zeros((T, DIM), torch.float32)
        q8x = zeros(T * nbx * 292, torch.uint8)
        q8h = zeros(P * nbh * 292, torch.uint8)
        h = zeros(P * FF, torch.float32)
        ints = zeros(P * rec, torch.int32)
        torch.cuda.synchronize()
        lane.grouped_trace_async(0, dev(ids), dev(w), dev(x), out, q8x, q8h, h, ints)
        lane.sync()
        q8x = q8x.cpu().numpy().reshape(T, -1)
        h, q8h, ints = h.cpu().numpy().reshape(P, FF), q8h.cpu().numpy().reshape(P, -1), ints.cpu().numpy().reshape(P, rec)
        got = out.cpu().numpy()
        mats = {}
        sig = (16, 16, 17)
        for t in range(T):
            want_q8x = check_q8x(orc, x[t], xs[t][1], q8x[t], f"token {t}")
            y64 = np.zeros(DIM)
            for i, e in enumerate(ids[t]):
                if int(e) not in mats:
                    mats[int(e)] = orc.gen_expert(sig, SEED, 0, int(e), DIM, FF)
                p = t * k + i
                tag = f"token {t} pick {i} (expert {e})"
                check_pick(orc, sig, mats[int(e)], DIM, FF, want_q8x, h[p], q8h[p], ints[p], tag)
                y64 += float(w[t, i]) * check_exact(sig, mats[int(e)], ints[p], want_q8x, h[p], q8h[p], tag)
            assert max_rel(got[t], y64) < TOL, t
    finally:
        lane.close()
