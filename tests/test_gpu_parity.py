"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars (the north star): Q8_K bytes and per-block int32 partials bit-exact;
f32 outputs within max relative error 1e-3 (max-norm, tests.conftest.max_rel);
runs bit-identical run to run. The hidden-state quantization is compared by
feeding the device's own SwiGLU output to the oracle quantizer (host and device
exp differ by ulps; the reference does the same, warm/expert_check.cpp:86-88).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

import crosslane_amd as xl
from oracle.oracle import BLOCK_BYTES
from tests.conftest import max_rel

pytestmark = pytest.mark.gpu
TOL = 1e-3

torch = pytest.importorskip("torch")


def step(msg):
    print(f"[gpu-step] {msg}", flush=True)
    sys.stdout.flush()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def types_map(L, E, gu, dn):
    t = np.zeros((L, E, 3), np.int32)
    t[..., 0] = gu; t[..., 1] = gu; t[..., 2] = dn
    return t


@pytest.fixture(scope="module")
def probe():
    """A context used only for primitives (quantize / matvec)."""
    lane = xl.Lane(4096, 4096, 1, 1, types_map(1, 1, 16, 16), max_picks=1)
    yield lane
    lane.close()


# ---- Q8_K -----------------------------------------------------------------------
def test_q8k_bit_exact(probe, orc, rng):
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))
    cases = [gold["q8k_x"].reshape(-1)]
    for scale in (1e-3, 1.0, 1e3):
        cases.append((rng.standard_normal(4096) * scale).astype(np.float32))
    for x in cases:
        step(f"q8k blocks={x.size // 256}")
        dx = dev(x.astype(np.float32))
        out = torch.zeros(x.size // 256 * 292, dtype=torch.uint8, device="cuda")
        probe.quantize_q8k_async(dx, 1, x.size, out)
        probe.sync()
        assert np.array_equal(out.cpu().numpy(), orc.quantize(x).view(np.uint8))


# ---- matvec + per-block partials -------------------------------------------------
@pytest.mark.parametrize("t", [16, 17, 29])
@pytest.mark.parametrize("n,k", [(64, 256), (96, 512), (40, 768), (128, 1024), (64, 2048), (48, 2304), (256, 3072),
                                 (256, 4096), (64, 5120)])
def test_matvec_partials_exact(probe, orc, t, n, k):
    step(f"matvec type={t} n={n} k={k}")
    aos = orc.gen_matrix(t, 1234 + k, 0, t, 0, n, k)
    planar = dev(xl.repack(t, n, k, aos))
    x = np.random.default_rng(n * k + t).standard_normal(k).astype(np.float32)
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    nb = k // 256
    parts = torch.zeros(n * nb, dtype=torch.int32, device="cuda")
    probe.matvec_async(t, planar, n, k, dev(x), y, parts)
    probe.sync()
    act = orc.quantize(x)
    rb = nb * BLOCK_BYTES[t]
    bp = np.stack([orc.block_partials(t, aos[r * rb:(r + 1) * rb], act) for r in range(n)])
    # one int per block; IQ1_M's (main, delta) enter as 8 * main + delta, the integer the decoder forms
    want_parts = (8 * bp[:, 0::2] + bp[:, 1::2]) if t == 29 else bp
    assert np.array_equal(parts.cpu().numpy(), want_parts.reshape(-1))
    want_y = orc.matvec(t, aos, n, k, act)
    assert max_rel(y.cpu().numpy(), want_y) < TOL


# ---- one expert, stage by stage ---------------------------------------------------
@pytest.mark.parametrize("dim,ff,sig", [(512, 256, (16, 16, 17)), (256, 768, (29, 29, 29)),
                                        (1024, 512, (17, 17, 16)), (4096, 3072, (16, 16, 17))])
def test_expert_stages(orc, dim, ff, sig):
    step(f"expert stages dim={dim} ff={ff} sig={sig}")
    E = 4
    lane = xl.Lane(dim, ff, 1, E, types_map(1, E, sig[0], sig[2]), max_picks=6)
    try:
        lane.generate(seed=0xABC)
        x = np.random.default_rng(dim + ff).standard_normal(dim).astype(np.float32)
        e = 2
        tr = lane.expert_trace(0, e, x)
        gate, up, down = orc.gen_expert(sig, 0xABC, 0, e, dim, ff)
        yo, go, uo, ho = orc.expert(sig, gate, up, down, dim, ff, x, intermediates=True)
        assert max_rel(tr["g"], go) < TOL and max_rel(tr["u"], uo) < TOL
        assert max_rel(tr["h"], ho) < TOL
        # Q8_K(h) bit-exact given the device's own h
        assert np.array_equal(tr["q8h"], orc.quantize(tr["h"]).view(np.uint8))
        # down from the device's h: partial-exact path, float within tolerance
        assert max_rel(tr["y"], orc.down_from_hidden(sig[2], down, dim, ff, tr["h"])) < TOL
        assert max_rel(tr["y"], yo) < TOL
    finally:
        lane.close()


# ---- generator -------------------------------------------------------------------
def test_device_generator_matches_oracle(orc):
    step("device generator")
    types = np.array([[[16, 16, 17], [29, 29, 29], [17, 17, 16]]], np.int32)
    lane = xl.Lane(512, 768, 1, 3, types, max_picks=3)
    try:
        lane.generate(seed=987654321)
        for e in range(3):
            for r in range(3):
                t = int(types[0, e, r])
                n, k = (768, 512) if r < 2 else (512, 768)
                assert np.array_equal(lane.download(0, e, r), orc.gen_matrix(t, 987654321, 0, e, r, n, k)), (e, r)
    finally:
        lane.close()


def test_upload_download_roundtrip(orc):
    step("upload/download")
    lane = xl.Lane(256, 256, 2, 2, types_map(2, 2, 29, 17), max_picks=2)
    try:
        aos = orc.gen_matrix(17, 5, 9, 9, 2, 256, 256)
        lane.upload(1, 1, 2, aos)
        assert np.array_equal(lane.download(1, 1, 2), aos)
    finally:
        lane.close()


# ---- layer: config-1 shapes --------------------------------------------------------
@pytest.fixture(scope="module")
def layer_lane():
    step("layer lane: 4096x3072, 384 experts, IQ2_XXS gate/up + IQ2_XS down")
    lane = xl.Lane(4096, 3072, 1, 384, types_map(1, 384, 16, 17), max_picks=8)
    lane.generate(seed=0x1A7E5)
    yield lane
    lane.close()


def route(logits, k=6):
    p = np.exp(logits - logits.max()); p /= p.sum()
    ids = np.argsort(-p, kind="stable")[:k]
    w = p[ids] / p[ids].sum()
    return ids.astype(np.int32), w.astype(np.float32)


def test_layer_vs_oracle(layer_lane, orc):
    rng = np.random.default_rng(11)
    for trial in range(2):
        ids, w = route(rng.standard_normal(384).astype(np.float32))
        x = rng.standard_normal(4096).astype(np.float32)
        shared = rng.standard_normal(4096).astype(np.float32) if trial else None
        step(f"layer trial={trial} ids={ids.tolist()}")
        got = layer_lane.layer_forward(0, ids, w, x, shared)
        rows = np.stack([orc.expert((16, 16, 17), *orc.gen_expert((16, 16, 17), 0x1A7E5, 0, int(e), 4096, 3072),
                                    4096, 3072, x) for e in ids])
        want = orc.combine(ids, w, rows, shared)
        assert max_rel(got, want) < TOL


def test_layer_deterministic_and_batch_equals_serial(layer_lane):
    rng = np.random.default_rng(12)
    ids, w = route(rng.standard_normal(384).astype(np.float32))
    x = rng.standard_normal(4096).astype(np.float32)
    step("layer determinism")
    a = layer_lane.layer_forward(0, ids, w, x)
    for _ in range(3):
        assert np.array_equal(a.view(np.uint32), layer_lane.layer_forward(0, ids, w, x).view(np.uint32))
    many = layer_lane.warm_compute_many(0, ids, x)
    for i, e in enumerate(ids):
        single = layer_lane.warm_compute(0, int(e), x)
        assert np.array_equal(single.view(np.uint32), many[i].view(np.uint32))


def test_layer_async_matches_sync(layer_lane):
    rng = np.random.default_rng(13)
    ids, w = route(rng.standard_normal(384).astype(np.float32))
    x = rng.standard_normal(4096).astype(np.float32)
    step("layer async")
    want = layer_lane.layer_forward(0, ids, w, x)
    out = torch.zeros(4096, dtype=torch.float32, device="cuda")
    layer_lane.layer_forward_async(0, dev(ids), dev(w), dev(x), out)
    layer_lane.sync()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_host_rejects_bad_routes(layer_lane):
    x = np.zeros(4096, np.float32)
    with pytest.raises(xl.XLError):
        layer_lane.layer_forward(0, [1, 1], [0.5, 0.5], x)
    with pytest.raises(xl.XLError):
        layer_lane.layer_forward(0, [384], [1.0], x)
    with pytest.raises(xl.XLError):
        layer_lane.layer_forward(0, [3], [1.0], np.full(4096, np.nan, np.float32))


@pytest.mark.parametrize("dim,ff,gu,dn,path", [(256, 256, 16, 16, "1"), (1024, 512, 16, 17, "1"),
                                               (4096, 3072, 16, 17, "1"), (4096, 3072, 29, 29, "1"),
                                               (4096, 3072, 16, 17, "3"), (5120, 2304, 16, 17, "1"),
                                               (5120, 2304, 29, 29, "1")])
def test_device_rejects_bad_id_and_poisons(monkeypatch, dim, ff, gu, dn, path):
    # An out-of-range id reaches the kernels only through the device path; the
    # kernels bounds-check it, skip the pick and raise the error flag (the
    # second to fourth cases run the streaming kernel, whose readers must still
    # finish; the last the all-types kernel).
    monkeypatch.setenv("XL_LAYER_PATH", path)
    step(f"device bad id dim={dim} ff={ff} types=({gu},{dn}) path={path}")
    lane = xl.Lane(dim, ff, 1, 4, types_map(1, 4, gu, dn), max_picks=2)
    try:
        lane.generate(1)
        out = torch.zeros(dim, dtype=torch.float32, device="cuda")
        lane.layer_forward_async(0, dev(np.array([1, 99], np.int32)), dev(np.array([0.5, 0.5], np.float32)),
                                 dev(np.ones(dim, np.float32)), out)
        with pytest.raises(xl.XLError, match="expert id"):
            lane.sync()
        with pytest.raises(xl.XLError, match="poisoned"):
            lane.layer_forward(0, [1], [1.0], np.ones(dim, np.float32))
    finally:
        lane.close()


@pytest.mark.parametrize("t", [16, 17, 29])
def test_matvec_any_fp16_scale(probe, orc, t):
    # Super-block scales over all finite fp16 classes: subnormal, negative, zero,
    # large. The device converts with the hardware f16->f32 instruction.
    n, k = 128, 1024
    step(f"matvec fp16 scales type={t}")
    rng = np.random.default_rng(t + 7)
    aos = orc.gen_matrix(t, 31, 0, 0, 0, n, k).reshape(-1, BLOCK_BYTES[t])
    h = rng.integers(0, 0x10000, size=aos.shape[0]).astype(np.uint16)
    h[(h & 0x7C00) == 0x7C00] &= 0xBFFF          # no inf/nan
    h[:16] = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00, 0xBC00, 0x0200, 0x83FF,
              0x1000, 0x9000, 0x2E66, 0x5555]
    if t == 29:
        for q in range(4):
            w = aos[:, 48 + 2 * q].astype(np.uint16) | (aos[:, 49 + 2 * q].astype(np.uint16) << 8)
            w = (w & 0x0FFF) | (((h >> (4 * q)) & 15) << 12)
            aos[:, 48 + 2 * q] = w & 0xFF; aos[:, 49 + 2 * q] = w >> 8
    else:
        aos[:, 0] = h & 0xFF; aos[:, 1] = h >> 8
    aos = aos.reshape(-1)
    x = rng.standard_normal(k).astype(np.float32)
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    probe.matvec_async(t, dev(xl.repack(t, n, k, aos)), n, k, dev(x), y)
    probe.sync()
    want = orc.matvec(t, aos, n, k, orc.quantize(x))
    got = y.cpu().numpy()
    assert np.all(np.isfinite(got))
    assert max_rel(got, want) < TOL


@pytest.mark.parametrize("dim,ff,sig", [(4096, 3072, None), (4096, 3072, (16, 16, 17)), (4096, 3072, (29, 29, 29)),
                                        (1024, 512, (17, 17, 16)),
                                        (1024, 512, (16, 16, 17)), (256, 768, (16, 16, 17)),
                                        (256, 768, (29, 29, 17)), (512, 256, (16, 16, 29)), (256, 256, (17, 17, 17))])
def test_layer_paths_agree(orc, dim, ff, sig, monkeypatch):
    # The single-launch kernels (path 1: the streaming kernel where one of its
    # instances fits the shape, else the all-types one; path 3: the all-types
    # one only), the separate launches (path 0) and the cooperative
    # kernel (path 2) share the row arithmetic per block but sum lanes in their
    # own orders, so they agree to the tolerance, and each is bit-identical run
    # to run; the oracle checks every path.
    step(f"layer paths dim={dim} ff={ff} sig={sig}")
    E, k = 24, 6
    rng = np.random.default_rng(dim * 7 + ff)
    if sig is None:   # config-3 style mix: per-expert types over the three formats
        t = rng.choice([16, 17, 29], size=E, p=[0.19, 0.17, 0.64]).astype(np.int32)
        types = np.stack([t, t, t], axis=-1)[None]
    else:
        types = types_map(1, E, sig[0], sig[2])
    lanes = {}
    extra = ("4",) if (dim, ff, sig) == (4096, 3072, (16, 16, 17)) else ()
    for path in ("1", "3", "0") + extra:
        monkeypatch.setenv("XL_LAYER_PATH", path)
        lanes[path] = xl.Lane(dim, ff, 1, E, types, max_picks=8)
        lanes[path].generate(seed=77)
    try:
        for trial in range(3):
            ids, w = route(rng.standard_normal(E).astype(np.float32), k)
            x = rng.standard_normal(dim).astype(np.float32)
            shared = rng.standard_normal(dim).astype(np.float32) if trial == 1 else None
            rows = []
            for e in ids:
                tt = tuple(int(v) for v in types[0, e])
                rows.append(orc.expert(tt, *orc.gen_expert(tt, 77, 0, int(e), dim, ff), dim, ff, x))
            want = orc.combine(ids, w, np.stack(rows), shared)
            for path, lane in lanes.items():
                got = lane.layer_forward(0, ids, w, x, shared)
                again = lane.layer_forward(0, ids, w, x, shared)
                assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), (path, trial)
                assert max_rel(got, want) < TOL, (path, trial, max_rel(got, want))
    finally:
        for lane in lanes.values():
            lane.close()


def kind_types(kind, E, seed=0):
    """Layer type maps by kind: IQ2_XXS gate/up + IQ2_XS down, IQ1_M only, or a
    per-expert mix of the three types (every type present)."""
    if kind == "iq2":
        return types_map(1, E, 16, 17)
    if kind == "iq1":
        return types_map(1, E, 29, 29)
    t = np.random.default_rng(seed + E).choice([16, 17, 29], size=E)
    t[:3] = [16, 17, 29]
    return np.repeat(t.reshape(1, E, 1), 3, axis=-1).astype(np.int32)


STREAM_CASES = [(4096, 3072, 6), (4096, 3072, 5), (4096, 3072, 4), (4096, 3072, 3), (4096, 3072, 2),
                (4096, 3072, 1), (1024, 512, 8), (1024, 512, 12), (1024, 512, 16), (256, 768, 6), (256, 768, 12),
                (5120, 2304, 6), (5120, 2304, 5), (5120, 2304, 4), (5120, 2304, 3), (5120, 2304, 2),
                (5120, 2304, 1)]
STREAM_CASES_OTHER = [(4096, 3072, 6), (4096, 3072, 4), (4096, 3072, 1), (1024, 512, 16), (256, 768, 12),
                      (5120, 2304, 6), (5120, 2304, 4), (5120, 2304, 1)]


@pytest.mark.parametrize("kind,dim,ff,k", [("iq2",) + c for c in STREAM_CASES] +
                         [(kd,) + c for kd in ("iq1", "mixed") for c in STREAM_CASES_OTHER])
def test_streaming_kernel_pick_counts(orc, kind, dim, ff, k, monkeypatch):
    # XL_LAYER_PATH=4 runs the streaming kernel or fails: pick counts that give
    # one, two or three down steps and steps staging one to eight picks must
    # match the oracle and repeat bit for bit, for the IQ2 instance, the IQ1_M
    # instance and the mixed-type instance (matrices from descriptors). At
    # 5120 x 2304 the single-type instances' down passes cross pick boundaries
    # (a workgroup's 20-row band of every pick, 16 rows a pass).
    step(f"streaming kernel {kind} dim={dim} ff={ff} k={k}")
    E = 24
    rng = np.random.default_rng(dim + ff + k)
    types = kind_types(kind, E)
    monkeypatch.setenv("XL_LAYER_PATH", "4")
    lane = xl.Lane(dim, ff, 1, E, types, max_picks=16)
    try:
        lane.generate(seed=91)
        for trial in range(2):
            ids, w = route(rng.standard_normal(E).astype(np.float32), k)
            x = rng.standard_normal(dim).astype(np.float32)
            shared = rng.standard_normal(dim).astype(np.float32) if trial else None
            rows = []
            for e in ids:
                sig = tuple(int(v) for v in types[0, e])
                rows.append(orc.expert(sig, *orc.gen_expert(sig, 91, 0, int(e), dim, ff), dim, ff, x))
            want = orc.combine(ids, w, np.stack(rows), shared)
            got = lane.layer_forward(0, ids, w, x, shared)
            again = lane.layer_forward(0, ids, w, x, shared)
            assert np.array_equal(got.view(np.uint32), again.view(np.uint32)), trial
            assert max_rel(got, want) < TOL, (trial, max_rel(got, want))
    finally:
        lane.close()


@pytest.mark.parametrize("limit", [0.0, 7.0])
def test_swiglu_primitive(probe, orc, rng, limit):
    """xl_swiglu_async (q8k::activate): the device's expf differs from the host's
    by an ulp or so, so the check is within 4 ulps; the clamp itself is exact."""
    step(f"swiglu limit={limit}")
    g = (rng.standard_normal(5000) * 8).astype(np.float32)
    u = (rng.standard_normal(5000) * 8).astype(np.float32)
    h = torch.zeros(5000, dtype=torch.float32, device="cuda")
    probe.swiglu_async(dev(g), dev(u), h, limit)
    probe.sync()
    want = np.array([orc.swiglu(a, b, limit) for a, b in zip(g, u)], np.float32)
    got = h.cpu().numpy()
    ulp = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert ulp.max() <= 4, ulp.max()
