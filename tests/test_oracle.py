"""CPU: pins the oracle (oracle/xl_oracle.c) before anything is compared with it.

Each function is checked against (a) the golden vectors written from the
reference's own q8k_core.hpp / other_combine.hpp (tests/golden), (b) the same
reference code compiled in oracle/_ref when present, and (c) what the
mathematics fixes: exact fp16 decode, closed-form Q8_K blocks, round-half-even
ties, a brute-force dequantize-and-multiply integer dot, and the reference's
independent per-32 decoder (sycl/moe/core.hpp:78-105).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle.oracle import BLOCK_BYTES, Q8K_DTYPE

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))


def f32bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---- scalars ------------------------------------------------------------------
def test_half_decode_exhaustive(orc):
    # q8k_core.hpp:17-24: every fp16 -> f32 exactly; numpy's float16 widening is exact.
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.lib.orc_half(int(v)) for v in h], dtype=np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(f32bits(got[finite]), f32bits(want[finite]))
    assert np.all(np.isnan(got[np.isnan(want)]))
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)])


def test_nearest_round_half_even(orc):
    # ggml nearest_int: round half to even for |x| < 2^22.
    for x, want in [(0.5, 0), (1.5, 2), (2.5, 2), (-0.5, 0), (-1.5, -2), (-2.5, -2), (126.5, 126), (127.49, 127),
                    (-127.0, -127), (3.0, 3)]:
        assert orc.lib.orc_nearest(x) == want, x


# ---- Q8_K -----------------------------------------------------------------------
def test_q8k_golden(orc):
    got = orc.quantize(GOLD["q8k_x"].reshape(-1)).view(np.uint8).reshape(-1, 292)
    assert np.array_equal(got, GOLD["q8k_bytes"])


def test_q8k_closed_forms(orc):
    z = orc.quantize(np.zeros(256, np.float32))[0]
    assert z["d"] == 0 and not z["qs"].any() and not z["bsums"].any()
    for c, j in [(3.5, 17), (-2.0, 0), (1e-20, 255)]:
        x = np.zeros(256, np.float32); x[j] = c
        b = orc.quantize(x)[0]
        # is = -127/c, so qs[j] = -127 and d = 1/is = -c/127 (rounded twice).
        assert b["qs"][j] == -127 and np.count_nonzero(b["qs"]) == 1
        assert b["d"] == np.float32(1.0) / (np.float32(-127.0) / np.float32(c))
        assert b["bsums"][j // 16] == -127
    # |max| tie: the FIRST value of largest magnitude sets the sign (strict '>').
    x = np.zeros(256, np.float32); x[5] = -4.0; x[9] = 4.0
    b = orc.quantize(x)[0]
    assert b["qs"][5] == -127 and b["qs"][9] == 127


def test_q8k_overflowing_inverse_scale(orc):
    # Largest magnitude below 127 / FLT_MAX: is = -127/mx overflows to -inf (mx > 0)
    # or +inf (mx < 0); nearest(+-inf) = -2^22 and nearest(NaN) = 0 both keep
    # the int8 byte 0 (q8k_core.hpp:25-29, 34), and d = 1/is = -0 / +0.
    for mx, dbits in [(1.0e-38, 0x80000000), (-1.0e-38, 0x00000000), (2.0e-39, 0x80000000)]:
        x = np.zeros(256, np.float32)
        x[::7] = np.float32(mx) * np.float32(0.25)
        x[100] = np.float32(mx)
        b = orc.quantize(x)[0]
        assert not b["qs"].any() and not b["bsums"].any(), mx
        assert np.float32(b["d"]).view(np.uint32) == dbits, mx
    # just above the threshold: is finite, and the block quantizes as usual
    x = np.zeros(256, np.float32); x[3] = np.float32(4.0e-37); x[4] = np.float32(-2.0e-37)
    b = orc.quantize(x)[0]
    assert b["qs"][3] == -127 and b["qs"][4] == 64 and np.isfinite(b["d"]) and b["d"] < 0


def test_q8k_overflow_vs_reference(orc, ref, rng):
    for mx in (1.0e-38, -1.0e-38, 3.0e-39, 3.7e-37, 3.8e-37):
        x = (rng.standard_normal(256) * abs(mx) * 0.3).astype(np.float32)
        x[int(rng.integers(256))] = np.float32(mx)
        assert orc.quantize(x).tobytes() == ref.quantize(x).tobytes(), mx


def test_q8k_vs_reference_random(orc, ref, rng):
    for scale in (1e-3, 1.0, 1e3):
        x = (rng.standard_normal(256 * 64) * scale).astype(np.float32)
        assert orc.quantize(x).tobytes() == ref.quantize(x).tobytes()


def test_q8k_bsums_and_range(orc, rng):
    x = rng.standard_normal(256 * 32).astype(np.float32)
    q = orc.quantize(x)
    assert np.all(q["qs"] >= -127) and np.all(q["qs"] <= 127)
    assert np.array_equal(q["bsums"], q["qs"].reshape(-1, 16, 16).astype(np.int32).sum(-1))
    # dequantized values within half a quantum of the input
    deq = q["qs"].astype(np.float64) * q["d"][:, None].astype(np.float64)
    err = np.abs(deq - x.reshape(-1, 256)) / np.abs(q["d"][:, None])
    assert err.max() <= 0.5 + 1e-3


# ---- IQ x Q8_K dot --------------------------------------------------------------
@pytest.mark.parametrize("t", [16, 17, 29])
def test_dot_golden(orc, t):
    act = orc.quantize(GOLD["dot_act_x"])
    rows = GOLD[f"dot{t}_rows"]
    got = np.array([orc.dot(t, rows[r], act) for r in range(rows.shape[0])], np.float32)
    assert np.array_equal(f32bits(got), f32bits(GOLD[f"dot{t}_y"]))
    bb = BLOCK_BYTES[t]
    for r in range(rows.shape[0]):
        for b in range(2):
            for l in range(8):
                assert orc.integer_lane(t, rows[r, b * bb:(b + 1) * bb], act[b:b + 1], l) == tuple(
                    GOLD[f"dot{t}_lanes"][r, b, l])


@pytest.mark.parametrize("t", [16, 17, 29])
def test_dot_vs_reference_generated(orc, ref, t):
    act = orc.quantize(np.random.default_rng(t).standard_normal(1024).astype(np.float32))
    w = orc.gen_matrix(t, 99, 3, 7, 1, 64, 1024)
    rb = 4 * BLOCK_BYTES[t]
    for r in range(64):
        row = w[r * rb:(r + 1) * rb]
        assert np.float32(orc.dot(t, row, act)).view(np.uint32) == np.float32(ref.dot(t, row, act)).view(np.uint32)


@pytest.mark.parametrize("t", [16, 17, 29])
def test_block_partials_brute_force(orc, t, rng):
    # The per-block integer is order-independent: a plain dequantize-and-multiply
    # pins it. IQ1_M's brute force is 8*main + delta (values 8*grid + delta).
    act = orc.quantize(rng.standard_normal(256 * 4).astype(np.float32))
    w = orc.gen_matrix(t, 5, 0, 1, 2, 16, 1024)
    bb = BLOCK_BYTES[t]
    for r in range(16):
        row = w[r * 4 * bb:(r + 1) * 4 * bb]
        parts = orc.block_partials(t, row, act)
        for b in range(4):
            brute = orc.brute_block(t, row[b * bb:(b + 1) * bb], act[b:b + 1])
            if t == 29:
                assert brute == 8 * parts[2 * b] + parts[2 * b + 1]
            else:
                assert brute == parts[b]


@pytest.mark.parametrize("t", [16, 17, 29])
def test_matrix_ints_brute_force(orc, t, rng):
    # orc_matrix_ints (the device trace's comparison target) against the
    # brute-force block dot, row by row, over several threads.
    n, k = 37, 1280
    act = orc.quantize(rng.standard_normal(k).astype(np.float32))
    w = orc.gen_matrix(t, 9, 1, 2, 1, n, k)
    got = orc.matrix_ints(t, w, n, k, act, threads=3)
    bb = BLOCK_BYTES[t]
    want = np.array([[orc.brute_block(t, w[(r * (k // 256) + b) * bb:(r * (k // 256) + b + 1) * bb], act[b:b + 1])
                      for b in range(k // 256)] for r in range(n)], np.int64)
    assert np.array_equal(got.astype(np.int64), want)


@pytest.mark.parametrize("t", [16, 17, 29])
def test_avx2_lane_rows_bit_identical(orc, t, rng):
    # The CPU baseline's AVX2 rows (cpu_lane.c) against the scalar AVX2-order
    # restatement, bit for bit, on generated rows and golden activations.
    if not orc.lane_avx2():
        pytest.skip("host without AVX2 + FMA")
    gold = np.load(os.path.join(os.path.dirname(__file__), "golden", "reference_vectors.npz"))
    k = 1024
    w = orc.gen_matrix(t, 21, 0, t, 1, 24, k)
    rb = (k // 256) * BLOCK_BYTES[t]
    acts = [orc.quantize(rng.standard_normal(k).astype(np.float32) * s) for s in (1e-3, 1.0, 1e3)]
    acts.append(orc.quantize(np.resize(gold["q8k_x"].reshape(-1), k).astype(np.float32)))
    for act in acts:
        for r in range(24):
            row = w[r * rb:(r + 1) * rb]
            assert np.float32(orc.lane_dot(t, row, act)).view(np.uint32) == np.float32(orc.dot(t, row, act)).view(np.uint32)


def test_avx2_lane_layer_bit_identical(orc, rng):
    # One routed layer on the AVX2 lane (threads, 64-row jobs, phases) equals the
    # scalar oracle's expert chain + fixed-order combine bit for bit.
    if not orc.lane_avx2():
        pytest.skip("host without AVX2 + FMA")
    dim, ff = 1024, 768
    sigs = [(16, 16, 17), (29, 29, 29), (17, 17, 16)]
    ids = np.array([5, 2, 9], np.int32)
    w = np.array([0.5, 0.3, 0.2], np.float32)
    x = rng.standard_normal(dim).astype(np.float32)
    mats = [orc.gen_expert(s, 3, 0, int(e), dim, ff) for s, e in zip(sigs, ids)]
    for limit in (0.0, 7.0):
        ph = np.zeros(5, np.float64)
        got = orc.lane_layer(np.array(sigs), mats, ids, w, x, dim, ff, threads=3, limit=limit, phases=ph)
        rows = np.stack([orc.expert(s, *m, dim, ff, x, limit=limit) for s, m in zip(sigs, mats)])
        want = orc.combine(ids, w, rows)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert np.all(ph[:4] > 0)


@pytest.mark.parametrize("t", [16, 17, 29])
def test_brute_force_vs_reference_decoder(orc, ref, t, rng):
    # Reference per-32 decoder (sycl/moe/core.hpp): values and odd sub-scales.
    w = orc.gen_matrix(t, 11, 1, 2, 0, 4, 256)
    bb = BLOCK_BYTES[t]
    x = rng.integers(-127, 128, size=256).astype(np.int8)
    act = np.zeros(1, dtype=Q8K_DTYPE); act["qs"][0] = x; act["d"] = 1.0
    for r in range(4):
        blk = w[r * bb:(r + 1) * bb]
        total = 0
        for kb in range(8):
            q, s, _ = ref.decode(t, blk, kb)
            total += int(s[0]) * int(np.dot(q[:16], x[32 * kb:32 * kb + 16].astype(np.int64)))
            total += int(s[1]) * int(np.dot(q[16:], x[32 * kb + 16:32 * kb + 32].astype(np.int64)))
        assert orc.brute_block(t, blk, act) == total


def test_dot_mutation_fails(orc):
    # A changed sign index must change the integer (a pin that can fail).
    act = orc.quantize(GOLD["dot_act_x"])
    rows = GOLD["dot16_rows"].copy()
    base = orc.block_partials(16, rows[1], act)
    rows[1, 2 + 4] ^= 0x01       # flip one sign bit of sub-block 0, group 0
    assert not np.array_equal(base, orc.block_partials(16, rows[1], act))


# ---- SwiGLU and combine -----------------------------------------------------------
def test_swiglu_golden(orc):
    g, u = GOLD["swiglu_gu"]
    for lim, key in ((0.0, "swiglu_y0"), (7.0, "swiglu_y7")):
        got = np.array([orc.swiglu(a, b, lim) for a, b in zip(g, u)], np.float32)
        assert np.array_equal(f32bits(got), f32bits(GOLD[key]))


def test_combine_golden(orc):
    i = 0
    while f"comb{i}_ids" in GOLD:
        got = orc.combine(GOLD[f"comb{i}_ids"], GOLD[f"comb{i}_w"], GOLD[f"comb{i}_rows"], GOLD[f"comb{i}_shared"])
        assert np.array_equal(f32bits(got), f32bits(GOLD[f"comb{i}_out"])), i
        i += 1
    assert i >= 5


def test_combine_order_matters(orc):
    # Ascending-id order is observable: a reordering that keeps ids fixed gives
    # identical bits, a different id order generally does not.
    rng = np.random.default_rng(3)
    rows = rng.standard_normal((6, 512)).astype(np.float32) * 1e3
    w = rng.random(6).astype(np.float32)
    ids = np.array([40, 3, 17, 200, 9, 100], np.int32)
    a = orc.combine(ids, w, rows)
    p = rng.permutation(6)
    assert np.array_equal(f32bits(a), f32bits(orc.combine(ids[p], w[p], rows[p])))
    sequential = np.zeros(512, np.float64)
    out = np.zeros(512, np.float32)
    for i in np.argsort(ids):
        out = (w[i].astype(np.float64) * rows[i].astype(np.float64) + out.astype(np.float64)).astype(np.float32)
    # float64 products of two floats are exact, so this is fma then one rounding.
    assert np.array_equal(f32bits(a), f32bits(out))


# ---- generator --------------------------------------------------------------------
def test_generator_fields(orc):
    for t in (16, 17, 29):
        w = orc.gen_matrix(t, 2026, 4, 9, 0, 64, 1024).reshape(-1, BLOCK_BYTES[t])
        if t == 29:
            sc = w[:, 48:56].view(np.uint16)
            d = ((sc[:, 0] >> 12) | ((sc[:, 1] >> 8) & 0xF0) | ((sc[:, 2] >> 4) & 0xF00) | (sc[:, 3] & 0xF000))
        else:
            d = w[:, 0:2].view(np.uint16)[:, 0]
        dv = d.astype(np.uint16).view(np.float16).astype(np.float64)
        assert dv.min() >= 1e-3 * (1 - 1e-3) and dv.max() <= 1e-2 * (1 + 1e-3)
        assert 0.4 < (dv.mean() - 1e-3) / 9e-3 < 0.6
        assert orc.gen_matrix(t, 2026, 4, 9, 0, 64, 1024).tobytes() == w.tobytes()  # pure function
        assert orc.gen_matrix(t, 2027, 4, 9, 0, 64, 1024).tobytes() != w.tobytes()


def test_codebook_self_consistency(orc):
    for which, vals in ((0, (8, 25, 43)), (1, (8, 25, 43)), (2, (0xFF, 0x00, 0x01))):
        cb = orc.codebook(which)
        b = cb.view(np.uint8)
        assert set(np.unique(b).tolist()) == set(vals)
        assert len(np.unique(cb)) == cb.size   # distinct rows
    ks = orc.ksigns()
    for i in range(128):
        assert ks[i] & 0x7F == i and bin(int(ks[i])).count("1") % 2 == 0


# ---- router (route.cpp:15-37) ------------------------------------------------
def test_route_golden(orc):
    for i in range(4):
        lg, b = GOLD[f"route{i}_logits"], GOLD[f"route{i}_bias"]
        k, scale = GOLD[f"route{i}_k_scale"]
        ids, w = orc.route(lg, int(k), float(scale), b)
        assert np.array_equal(ids, GOLD[f"route{i}_ids"]), i
        assert np.array_equal(w.view(np.uint32), GOLD[f"route{i}_w"].view(np.uint32)), i


def test_route_vs_reference_random(orc, ref, rng):
    for T, n, k, s in ((32, 384, 6, 1.0), (8, 4096, 8, 2.5), (3, 7, 7, 0.0)):
        lg = (rng.standard_normal((T, n)) * rng.choice([0.5, 4.0, 40.0])).astype(np.float32)
        b = (rng.standard_normal(n) * 0.3).astype(np.float32)
        a, c = orc.route(lg, k, s, b), ref.route(lg, k, s, b)
        assert np.array_equal(a[0], c[0])
        assert np.array_equal(a[1].view(np.uint32), c[1].view(np.uint32))


def test_route_independent_forms(orc, rng):
    # With no bias the key sqrt(softplus(l)) is increasing in l: the picks are
    # the stable descending order of the logits. The weights against a float64
    # restatement of score / sum(scores) * scale.
    lg = rng.standard_normal((40, 384)).astype(np.float32)
    ids, w = orc.route(lg, 6, 1.75)
    for t in range(40):
        assert np.array_equal(ids[t], np.argsort(-lg[t], kind="stable")[:6])
        sc = np.sqrt(np.log1p(np.exp(lg[t, ids[t]].astype(np.float64))))
        np.testing.assert_allclose(w[t], sc / sc.sum() * 1.75, rtol=2e-6)
    # equal keys: the first index wins; k = n picks every expert once
    ids, _ = orc.route(np.array([[2.0, 5.0, 5.0, 5.0]], np.float32), 2)
    assert ids.tolist() == [[1, 2]]
    ids, w = orc.route(rng.standard_normal((3, 9)).astype(np.float32), 9, 1.0)
    assert all(sorted(r) == list(range(9)) for r in ids.tolist())
    np.testing.assert_allclose(w.sum(axis=1), 1.0, rtol=1e-6)
    # above 20 the score is sqrt(l) itself
    ids, w = orc.route(np.array([[30.0, 25.0]], np.float32), 2)
    np.testing.assert_allclose(w[0], np.sqrt([30.0, 25.0]) / np.sqrt([30.0, 25.0]).sum(), rtol=1e-6)


# ---- per32 arithmetic (the production HIP lane) -------------------------------
def test_quant32_closed_forms(orc, rng):
    x = np.zeros(96, np.float32)
    x[40] = -3.5                                   # one-hot in block 1
    x[64:96] = np.arange(32, dtype=np.float32) - 10.5   # ramp with .5 fractions in block 2
    q, d = orc.quant32(x)
    assert (q[:32] == 0).all() and d[0] == 0.0
    assert q[40] == -127 and np.float32(d[1]) == np.float32(3.5) / np.float32(127.0)
    assert (q[32:40] == 0).all() and (q[41:64] == 0).all()
    want = np.rint((x[64:96] / d[2]).astype(np.float32)).astype(np.int8)   # np.rint: half to even
    assert np.array_equal(q[64:96], want) and abs(q[64:96]).max() == 127
    x = (rng.standard_normal(32 * 64) * rng.choice([1e-3, 1.0, 1e3])).astype(np.float32)
    q, d = orc.quant32(x)
    err = np.abs(x - q.astype(np.float64) * np.repeat(d, 32))
    assert (err <= np.repeat(d, 32) * 0.5000001).all()


def test_row32_golden(orc):
    for t in (16, 17, 29):
        for k in (1024, 4096):
            q, d, rows = GOLD[f"row32_{t}_{k}_q"], GOLD[f"row32_{t}_{k}_d"], GOLD[f"row32_{t}_{k}_rows"]
            got = np.array([orc.row32(t, rows[r], k, q, d) for r in range(4)], np.float32)
            assert np.array_equal(got.view(np.uint32), GOLD[f"row32_{t}_{k}_y"].view(np.uint32)), (t, k)


@pytest.mark.parametrize("t", [16, 17, 29])
def test_row32_vs_reference_and_float64(orc, ref, t, rng):
    for k in (256, 3072, 4096):
        x = rng.standard_normal(k).astype(np.float32)
        q, d = orc.quant32(x)
        rows = orc.gen_matrix(t, 77, 1, 2, 0, 6, k).reshape(6, -1)
        for r in range(6):
            y = orc.row32(t, rows[r], k, q, d)
            assert np.float32(y).view(np.uint32) == np.float32(ref.row32(t, rows[r], k, q, d)).view(np.uint32)
        # independent of the float order: a float64 sum over the reference's own
        # per-32 decoder (values, odd half scales, d / 8)
        w = orc.matvec32(t, rows.reshape(-1), 6, k, q, d)
        for r in range(6):
            tot = 0.0
            for kb in range(k // 32):
                vals, sc, d8 = ref.decode(t, rows[r], kb)
                qq = q[32 * kb:32 * kb + 32].astype(np.int64)
                i = sc[0] * int(np.dot(vals[:16], qq[:16])) + sc[1] * int(np.dot(vals[16:], qq[16:]))
                tot += float(d[kb]) * float(d8) * i
            assert abs(w[r] - tot) <= 2e-5 * (abs(tot) + 1e-3), (r, w[r], tot)


@pytest.mark.parametrize("limit", [0.0, 1.0, 7.0])
def test_expert_chain_vs_reference_with_limit(orc, ref, rng, limit):
    """The Q8_K expert chain with the SwiGLU limit (model_meta.hpp:34 lim):
    bit-identical to the reference's own functions; the limit must bite."""
    t3, dim, ff = (16, 16, 17), 1024, 512
    mats = orc.gen_expert(t3, 5, 0, 3, dim, ff)
    x = rng.standard_normal(dim).astype(np.float32)
    y, g, u, h = orc.expert(t3, *mats, dim, ff, x, intermediates=True, limit=limit)
    assert np.array_equal(y.view(np.uint32), ref.expert(t3, *mats, dim, ff, x, limit=limit).view(np.uint32))
    if limit > 0:
        assert (np.abs(g) > limit).any() or (np.abs(u) > limit).any()
        assert not np.array_equal(y, orc.expert(t3, *mats, dim, ff, x))
        want = [orc.swiglu(min(a, limit), min(max(b, -limit), limit)) for a, b in zip(g, u)]
        assert np.array_equal(h, np.array(want, np.float32))


# ---- per32 dense formats (shared-expert matrices) and hc_post ------------------
@pytest.mark.parametrize("t", [8, 12, 13, 14])
def test_row32_dense_vs_reference_and_float64(orc, ref, t, rng):
    from tests.dense import dense_matrix
    for k in (256, 1024, 4096):
        x = (rng.standard_normal(k) * 3.0).astype(np.float32)
        q, d = orc.quant32(x)
        n = 5
        w = dense_matrix(t, n, k, seed=k)
        rb = orc.row_bytes32(t, k)
        assert w.size == n * rb
        y = orc.matvec32(t, w, n, k, q, d)
        for r in range(n):
            row = w[r * rb:(r + 1) * rb]
            assert np.float32(y[r]).view(np.uint32) == np.float32(ref.row32(t, row, k, q, d)).view(np.uint32), (t, k, r)
            tot = 0.0
            for kb in range(k // 32):
                vals, sc, dd, mm = ref.decode_full(t, row, kb)
                deq = (float(dd) * vals.astype(np.float64) if t == 8 else
                       float(dd) * np.repeat(sc, 16) * vals - np.repeat(mm.astype(np.float64), 16))
                assert np.allclose(orc.dequant32(t, row, kb), deq, rtol=1e-12, atol=0), (t, kb)
                tot += float(d[kb]) * float(np.dot(deq, q[32 * kb:32 * kb + 32]))
            assert abs(y[r] - tot) <= 2e-5 * (np.abs(y).max() + 1e-3), (t, k, r, y[r], tot)


def test_row32_dense_golden(orc):
    for t in (8, 12, 13, 14):
        q, d, rows = GOLD[f"row32_{t}_1024_q"], GOLD[f"row32_{t}_1024_d"], GOLD[f"row32_{t}_1024_rows"]
        got = np.array([orc.row32(t, rows[r], 1024, q, d) for r in range(rows.shape[0])], np.float32)
        assert np.array_equal(got.view(np.uint32), GOLD[f"row32_{t}_1024_y"].view(np.uint32)), t


def test_hc_post_reference_golden_and_closed_form(orc, ref, rng):
    T, H, D = 3, 4, 96
    y = rng.standard_normal((T, D)).astype(np.float32)
    res = rng.standard_normal((T, H, D)).astype(np.float32)
    post = rng.random((T, 8)).astype(np.float32) * 2
    comb = rng.random((T, 64)).astype(np.float32)
    got = orc.hc_post(y, res, post, comb, D, H, T)
    assert np.array_equal(got.view(np.uint32), ref.hc_post(y, res, post, comb, D, H, T).view(np.uint32))
    g = {k: GOLD[f"hc_{k}"] for k in ("y", "res", "post", "comb", "out")}
    Tg, Hg, Dg = g["out"].shape
    assert np.array_equal(orc.hc_post(g["y"], g["res"], g["post"], g["comb"], Dg, Hg, Tg).view(np.uint32),
                          g["out"].view(np.uint32))
    # post = 1, comb = identity: out[k] = y + res[k], one rounding
    eye = np.zeros((T, 64), np.float32)
    for k in range(H):
        eye[:, k * H + k] = 1.0
    out = orc.hc_post(y, res, np.ones((T, 8), np.float32), eye, D, H, T)
    assert np.array_equal(out, (y[:, None, :] + res).astype(np.float32))
    # a transposed comb (k * H + j) gives a different answer
    assert not np.array_equal(got, orc.hc_post(y, res, post, _transpose_comb(comb, H), D, H, T))


def test_hc_pre_norm_reference_golden_and_closed_form(orc, ref, rng):
    # sycl/hc/core.hpp:74-80: against the reference build and its golden vectors
    for D, H, T in ((4096, 1, 1), (5120, 4, 2), (1500, 3, 2), (7, 2, 1), (1024, 4, 1)):
        h = (rng.standard_normal((T, H, D)) * rng.choice([1e-3, 1.0, 40.0])).astype(np.float32)
        h[0, 0, : min(D, 3)] = -0.0   # 0 + (-0) = +0 in the reference's sum
        mix = rng.standard_normal((T, 8)).astype(np.float32)
        w = rng.standard_normal(D).astype(np.float32)
        for ww in (None, w):
            got = orc.hc_pre_norm(h, mix, ww)
            assert np.array_equal(got.view(np.uint32), ref.hc_pre_norm(h, mix, ww).view(np.uint32)), (D, H, T)
    g = {k: GOLD[f"hcpre_{k}"] for k in ("h", "mix", "w", "x")}
    assert np.array_equal(orc.hc_pre_norm(g["h"], g["mix"], g["w"]).view(np.uint32), g["x"].view(np.uint32))
    # one stream, mix 1, no weight: x = h exactly, with +0 for -0
    h = rng.standard_normal((2, 1, 3000)).astype(np.float32)
    h[0, 0, 5] = -0.0
    one = np.ones((2, 8), np.float32)
    x = orc.hc_pre_norm(h, one, None)
    assert np.array_equal(x, h[:, 0, :]) and not np.signbit(x[0, 5])
    # with a unit weight: x / sqrt(mean(x^2) + eps), to float rounding
    xn = orc.hc_pre_norm(h, one, np.ones(3000, np.float32))
    want = h[:, 0, :] / np.sqrt((h[:, 0, :].astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    assert np.allclose(xn, want, rtol=1e-5, atol=0)
    # all zeros: x = 0 (inv = 1 / sqrt(eps))
    assert not orc.hc_pre_norm(np.zeros((1, 2, 64), np.float32), one[:1], np.ones(64, np.float32)).any()
    # a dropped stream (mix of the last stream ignored) changes the answer
    h4 = rng.standard_normal((1, 4, 256)).astype(np.float32)
    m4 = rng.standard_normal((1, 8)).astype(np.float32)
    assert not np.array_equal(orc.hc_pre_norm(h4, m4, None), orc.hc_pre_norm(h4[:, :3], m4, None))


def _transpose_comb(comb, H):
    c = comb.copy()
    for j in range(H):
        for k in range(H):
            c[:, j * H + k] = comb[:, k * H + j]
    return c
