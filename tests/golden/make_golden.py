"""Writes tests/golden/reference_vectors.npz from the reference's own CPU code.

The reference's q8k_core.hpp / other_combine.hpp are compiled from
/root/reference into oracle/_ref/libxlref.so (oracle/Makefile); this script
calls that build on seeded inputs and stores inputs + outputs as plain arrays.
Run in the development container only (the GPU box has no reference tree):

    make -C oracle && python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle.oracle import BLOCK_BYTES, Q8K_DTYPE, Reference  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_vectors.npz")


def q8k_inputs(rng):
    blocks = [rng.standard_normal(256).astype(np.float32) for _ in range(6)]
    z = np.zeros(256, np.float32); blocks.append(z)
    neg = np.zeros(256, np.float32); neg[-0 + 17] = -3.5; blocks.append(neg)                # one-hot negative
    tie = np.full(256, 0.5, np.float32); tie[3] = -127.0; blocks.append(tie)                 # x*is lands on .5 ties
    dup = rng.standard_normal(256).astype(np.float32); dup[40] = 9.0; dup[200] = -9.0; blocks.append(dup)  # |max| tie
    tiny = (rng.standard_normal(256) * 1e-39).astype(np.float32); blocks.append(tiny)       # subnormal inputs
    big = (rng.standard_normal(256) * 1e30).astype(np.float32); blocks.append(big)
    ramp = np.arange(256, dtype=np.float32) - 128.0; blocks.append(ramp)
    return np.stack(blocks)


def main():
    ref = Reference()
    rng = np.random.default_rng(0x5EED)
    out = {}
    x = q8k_inputs(rng)
    out["q8k_x"] = x
    out["q8k_bytes"] = ref.quantize(x.reshape(-1)).view(np.uint8).reshape(x.shape[0], 292)
    # IQ x Q8_K dots: 3 types, rows of 2 blocks (k = 512), AVX2-order floats and lane integers.
    act_x = rng.standard_normal(512).astype(np.float32)
    act = ref.quantize(act_x)
    out["dot_act_x"] = act_x
    for t in (16, 17, 29):
        bb = BLOCK_BYTES[t]
        rows = rng.integers(0, 256, size=(8, 2 * bb), dtype=np.uint8)
        for r in range(8):
            for b in range(2):  # finite fp16 super-block scales
                h = np.float16(rng.uniform(1e-3, 1e-2) * (-1 if r % 3 == 0 else 1)).view(np.uint16)
                blk = rows[r, b * bb:(b + 1) * bb]
                if t != 29:
                    blk[0] = h & 0xFF; blk[1] = h >> 8
                else:
                    for q in range(4):
                        w = int(blk[48 + 2 * q]) | (int(blk[49 + 2 * q]) << 8)
                        w = (w & 0x0FFF) | (((int(h) >> (4 * q)) & 15) << 12)
                        blk[48 + 2 * q] = w & 0xFF; blk[49 + 2 * q] = w >> 8
        out[f"dot{t}_rows"] = rows
        out[f"dot{t}_y"] = np.array([ref.dot(t, rows[r], act) for r in range(8)], np.float32)
        lanes = np.zeros((8, 2, 8, 2), np.int32)
        for r in range(8):
            for b in range(2):
                for l in range(8):
                    lanes[r, b, l] = ref.integer_lane(t, rows[r, b * bb:(b + 1) * bb], act[b:b + 1], l)
        out[f"dot{t}_lanes"] = lanes
    # SwiGLU samples (limit 0 and 7).
    g = np.concatenate([rng.standard_normal(64) * 6, [0.0, -0.0, 80.0, -80.0, 1e-30]]).astype(np.float32)
    u = rng.standard_normal(g.size).astype(np.float32)
    out["swiglu_gu"] = np.stack([g, u])
    out["swiglu_y0"] = np.array([ref.swiglu(a, b, 0.0) for a, b in zip(g, u)], np.float32)
    out["swiglu_y7"] = np.array([ref.swiglu(a, b, 7.0) for a, b in zip(g, u)], np.float32)
    # Fixed-order combine with signed zeros and denormals (other_combine_check.cpp:30-39 style).
    cases = []
    for dim, k in ((1, 1), (7, 3), (257, 6), (4096, 6), (64, 16)):
        bits = rng.integers(0, 2**32, size=(k + 2, dim), dtype=np.uint64).astype(np.uint32)
        bits = (bits & np.uint32(0x807FFFFF)) | ((rng.integers(0, 190, size=bits.shape).astype(np.uint32)) << 23)
        vals = bits.view(np.float32).copy()
        rows = vals[:k].copy(); rows[:, 0] = np.where(np.arange(k) % 2, -0.0, 0.0)
        if dim > 1:
            rows[:, 1] = (np.arange(k, dtype=np.uint32) + 1).view(np.float32)
        ids = rng.permutation(384)[:k].astype(np.int32)
        w = vals[k, :k].copy() if dim >= k else rng.standard_normal(k).astype(np.float32)
        shared = vals[k + 1].copy()
        cases.append((ids, w, rows, shared, ref.combine(ids, w, rows, shared)))
    for i, (ids, w, rows, shared, y) in enumerate(cases):
        out[f"comb{i}_ids"], out[f"comb{i}_w"], out[f"comb{i}_rows"] = ids, w, rows
        out[f"comb{i}_shared"], out[f"comb{i}_out"] = shared, y
    # Router (route.cpp:15-37): N(0,1) logits, the softplus cut at 20, very
    # negative logits, bias on and off, equal keys (first index wins), k = n.
    rcases = []
    lg = rng.standard_normal((16, 384)).astype(np.float32)
    rcases.append((lg, np.zeros(384, np.float32), 6, 1.0))
    lg = (rng.standard_normal((8, 384)) * 15).astype(np.float32)
    lg[:, :8] = np.array([19.99, 20.0, 20.01, 25.0, -90.0, -200.0, 0.0, -0.0], np.float32)
    rcases.append((lg, (rng.standard_normal(384) * 0.2).astype(np.float32), 8, 2.5))
    lg = np.tile(np.array([1.0, 3.0, 3.0, 2.0, 3.0, -1.0], np.float32), (2, 1))
    rcases.append((lg, np.array([0.0, 0.0, 0.0, 0.0, 0.0, 5.0], np.float32), 3, 1.0))
    lg = rng.standard_normal((4, 16)).astype(np.float32)
    rcases.append((lg, np.zeros(16, np.float32), 16, 0.5))
    for i, (lg, b, k, scale) in enumerate(rcases):
        ids, w = ref.route(lg, k, scale, b)
        out[f"route{i}_logits"], out[f"route{i}_bias"] = lg, b
        out[f"route{i}_k_scale"] = np.array([k, scale], np.float32)
        out[f"route{i}_ids"], out[f"route{i}_w"] = ids, w
    # per32 rows (sycl/moe/core.hpp lane<> + the expert_check.cpp:50-55 butterfly):
    # 4 rows per type at k = 1024 and 4096 against per-32 quantized N(0,1) activations.
    from oracle.oracle import Oracle   # the per-32 quantizer has no CPU reference function to call
    orc = Oracle()
    for t in (16, 17, 29):
        for k in (1024, 4096):
            x = rng.standard_normal(k).astype(np.float32)
            q, d = orc.quant32(x)
            rows = orc.gen_matrix(t, 0x32, 0, 0, 0, 4, k).reshape(4, -1)
            out[f"row32_{t}_{k}_q"], out[f"row32_{t}_{k}_d"], out[f"row32_{t}_{k}_rows"] = q, d, rows
            out[f"row32_{t}_{k}_y"] = np.array([ref.row32(t, rows[r], k, q, d) for r in range(4)], np.float32)
    # per32 rows of the dense shared-expert formats (Q8_0, Q4_K, Q5_K, Q6_K) at
    # k = 1024 (own generator, so the vectors above keep their values).
    from tests.dense import dense_matrix
    rng2 = np.random.default_rng(0xD3)
    for t in (8, 12, 13, 14):
        k = 1024
        x = (rng2.standard_normal(k) * 2.0).astype(np.float32)
        q, d = orc.quant32(x)
        rows = dense_matrix(t, 4, k, seed=t).reshape(4, -1)
        out[f"row32_{t}_{k}_q"], out[f"row32_{t}_{k}_d"], out[f"row32_{t}_{k}_rows"] = q, d, rows
        out[f"row32_{t}_{k}_y"] = np.array([ref.row32(t, rows[r], k, q, d) for r in range(4)], np.float32)
    # hyper-connection post (sycl/hc/core.hpp:81-86): T = 2 tokens, H = 4 streams, D = 64
    T, H, D = 2, 4, 64
    hy = rng2.standard_normal((T, D)).astype(np.float32)
    hres = rng2.standard_normal((T, H, D)).astype(np.float32)
    hpost = (rng2.random((T, 8)) * 2).astype(np.float32)
    hcomb = rng2.random((T, 64)).astype(np.float32)
    out["hc_y"], out["hc_res"], out["hc_post"], out["hc_comb"] = hy, hres, hpost, hcomb
    out["hc_out"] = ref.hc_post(hy, hres, hpost, hcomb, D, H, T)
    # hyper-connection pre + RMS norm (sycl/hc/core.hpp:74-80): T = 2, H = 4, D = 1500
    T, H, D = 2, 4, 1500
    ph = rng2.standard_normal((T, H, D)).astype(np.float32)
    pmix = rng2.standard_normal((T, 8)).astype(np.float32)
    pw = rng2.standard_normal(D).astype(np.float32)
    out["hcpre_h"], out["hcpre_mix"], out["hcpre_w"] = ph, pmix, pw
    out["hcpre_x"] = ref.hc_pre_norm(ph, pmix, pw, 1e-6)
    np.savez_compressed(OUT, **out)
    print("wrote", OUT, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
