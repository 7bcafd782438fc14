#!/usr/bin/env python3
"""Routed-expert benchmark on one MI355X.

Default workload (benchmark config 1): one MoE layer at decode batch 1, d_model
4096, d_ff 3072, 384 resident experts (gate/up IQ2_XXS, down IQ2_XS), top-6 of
a softmax over seeded N(0,1) router logits with renormalized weights,
fixed-order combine into a 4096-wide f32 output. A step is one layer call
through the C ABI (xl_layer_forward_async) with routes, inputs and the bank
already resident in HBM; every step uses a fresh seeded route so consecutive
steps touch different experts (the bank is ~3.9 GB, far beyond the 256 MB MALL).

--config selects the other single-GPU workloads of the same metric:
  0  one config-1 expert per step (k = 1, w = 1), fresh expert each step;
  2  all-IQ1_M bank, 6 distinct experts drawn with p ~ rank^-1.1 over a seeded
     permutation (Zipf: hot experts recur, so the MALL can serve part of it);
  4  grouped: 512 tokens per step, each with its own top-6 of 384 config-1
     experts (xl_grouped_forward_async: every touched expert read once per 16
     of its pairs, int8 MFMA);
  3  a 40-layer pass per step: 40 x 384 experts whose whole-expert type is
     drawn 17 % IQ2_XS / 19 % IQ2_XXS / 64 % IQ1_M, top-6 per layer, the
     hidden carried layer to layer through an RMS normalization (the library's
     hyper-connection pre + RMS norm with one stream and a unit weight, inside
     each next layer's launch, xl_layer_forward_prenorm_async, and after the
     last layer by xl_hc_pre_norm_async, all inside the timed region: the
     model's ffn_norm step, without which the quadratic SwiGLU overflows f32
     within a few layers);
  6  config 1 at the real model's expert shape: d_model 5120, d_ff 2304
     (engine/strata/fixtures/moe/cpu_lane_fixture.cpp:17), the model's SwiGLU
     limit 10, 384 resident experts, top-6.

Prints one JSON line: value = achieved algorithmic HBM GB/s (selected experts'
weight bytes + x in + out per layer), plus us_per_layer; the roofline of the
layer kernel (one launch per layer, so its average duration is the timed
region's HIP-event time on the launching stream divided by the launches; HBM
traffic per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
summary in profiles/, config 1); and the CPU baseline (the AVX2 restatement of
the reference CPU lane in oracle/cpu_lane.c, bit-identical to the scalar
restatement, at 1 worker and at the box's CPU share with its phase split, and
the reference's own scalar q8k_core.hpp chain from oracle/_ref beside it, on a
bounded sample on the host cores).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

DIM, FF, E, K = 4096, 3072, 384, 6
REAL_DIM, REAL_FF, REAL_LIM = 5120, 2304, 10.0   # config 6: the DeepSeek expert shape and SwiGLU limit
GATE_T, DOWN_T = 16, 17
BYTES = {16: 66, 17: 74, 29: 56}
W_GU = FF * (DIM // 256) * BYTES[GATE_T]          # 3,244,032 B per gate/up matrix
W_DN = DIM * (FF // 256) * BYTES[DOWN_T]          # 3,637,248 B per down matrix
LAYER_BYTES = K * (2 * W_GU + W_DN) + 2 * DIM * 4  # 60,784,640 B
HBM_PEAK_GBS = 8000.0
SEED = 0x1A7E5
PMC_SUMMARY = os.path.join(ROOT, "profiles", "stream_kernel_config1_hbm_traffic.md")
N_LAYERS_3 = 40
MIX_3 = ((17, 0.17), (16, 0.19), (29, 0.64))   # whole-expert type draw of config 3


def expert_bytes(t3) -> int:
    """Weight bytes of one expert with (gate, up, down) types t3."""
    return FF * (DIM // 256) * (BYTES[t3[0]] + BYTES[t3[1]]) + DIM * (FF // 256) * BYTES[t3[2]]


SHARED_T = (13, 13, 14)    # config 5 shared expert: Q5_K gate/up, Q6_K down (the pack's K-quants)
DENSE_BYTES = {8: 34, 12: 144, 13: 176, 14: 210}
DENSE_VALUES = {8: 32, 12: 256, 13: 256, 14: 256}
HC_H = 4                   # hyper-connection streams


def dense_bytes(t, n, k) -> int:
    return n * (k // DENSE_VALUES[t]) * DENSE_BYTES[t]


def block_extra_bytes() -> int:
    """Config 5: what the MoE block reads and writes beyond the routed layer's
    bytes: the shared expert's gate and up (FF x DIM) and down (DIM x FF) in
    SHARED_T, hc_post's residual streams in and post streams out (HC_H x DIM
    floats each), post (8) and comb (64)."""
    return (dense_bytes(SHARED_T[0], FF, DIM) + dense_bytes(SHARED_T[1], FF, DIM)
            + dense_bytes(SHARED_T[2], DIM, FF) + 2 * HC_H * DIM * 4 + 72 * 4)


def dense_matrix(t, n, k, rng):
    """Uniform random ggml blocks of a dense format with finite fp16 scales in [1e-3, 1e-2)."""
    nb = n * (k // DENSE_VALUES[t])
    blk = rng.integers(0, 256, size=(nb, DENSE_BYTES[t]), dtype=np.uint8)
    for off in {8: (0,), 12: (0, 2), 13: (0, 2), 14: (208,)}[t]:
        blk[:, off:off + 2] = rng.uniform(1e-3, 1e-2, nb).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def measured_traffic():
    """HBM bytes per layer launch from the committed counter summary, or None."""
    try:
        for line in open(PMC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def routes(n, seed):
    rng = np.random.default_rng(seed)
    ids = np.zeros((n, K), np.int32)
    w = np.zeros((n, K), np.float32)
    for i in range(n):
        logits = rng.standard_normal(E).astype(np.float32)
        p = np.exp(logits - logits.max()).astype(np.float64)
        p /= p.sum()
        top = np.argsort(-p, kind="stable")[:K]
        ids[i] = top
        w[i] = (p[top] / p[top].sum()).astype(np.float32)
    x = rng.standard_normal((n, DIM)).astype(np.float32)
    return ids, w, x


def zipf_routes(n, seed, s=1.1):
    """Config 2: K distinct experts drawn without replacement with p ~ rank^-s
    over a seeded permutation of the experts; weights = renormalized p."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    p_rank = np.arange(1, E + 1, dtype=np.float64) ** -s
    p = np.zeros(E)
    p[perm] = p_rank / p_rank.sum()
    ids = np.zeros((n, K), np.int32)
    w = np.zeros((n, K), np.float32)
    for i in range(n):
        pick = rng.choice(E, size=K, replace=False, p=p)
        ids[i] = pick
        w[i] = (p[pick] / p[pick].sum()).astype(np.float32)
    x = rng.standard_normal((n, DIM)).astype(np.float32)
    return ids, w, x


def mixed_types(n_layers, seed):
    """Config 3: per (layer, expert) one type for all three matrices."""
    rng = np.random.default_rng(seed)
    tv = np.array([t for t, _ in MIX_3], np.int32)
    t = rng.choice(tv, size=(n_layers, E), p=[p for _, p in MIX_3])
    return np.repeat(t[..., None], 3, axis=-1).astype(np.int32)


def host_info():
    """Host CPU model, physical cores and logical CPUs this process may use, ISA."""
    model, cores, flags = "unknown", set(), set()
    allowed = os.sched_getaffinity(0)
    try:
        cpu, phys, core = None, None, None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                cpu = int(v)
            elif k == "model name" and model == "unknown":
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
                if cpu in allowed:
                    cores.add((phys, core))
            elif k == "flags" and not flags:
                flags = set(v.split())
    except OSError:
        pass
    isa = [f for f in ("avx2", "fma", "avx512f", "avx512bw", "avx512_vnni") if f in flags]
    return {"cpu": model, "physical_cores": len(cores) or len(allowed), "logical_cpus": len(allowed),
            "isa_present": isa}


def cpu_baseline(budget_s: float = 12.0, pool: int = 48, config: int = 1, max_threads: int = 0):
    """The CPU baseline: this repo's AVX2 restatement of the reference CPU lane
    (oracle/cpu_lane.c: ggml's AVX2 lane and FMA order, bit-identical to the
    scalar restatement; 64-row jobs, phases q1 / gate_up / q2 / down,
    engine/strata/sycl/moe/cpu_lane.cpp:70-81,157-170), at 1 worker and at the
    box's CPU share (physical cores, capped at the share), plus the reference's
    own scalar q8k_core.hpp chain (oracle/_ref) on a few layers, labelled.

    The picks are drawn from a pool of `pool` generated experts (48 x ~9 MB,
    beyond the host caches) typed as the config's; generation is not timed."""
    from oracle.oracle import Oracle, Reference   # checker/baseline only
    orc = Oracle()
    host = host_info()
    share = max_threads or int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or min(16, host["logical_cpus"])
    workers = sorted({1, min(host["physical_cores"], share), min(host["logical_cpus"], share)})
    rng = np.random.default_rng(SEED + 1)
    if config == 2:
        ptypes = [(29, 29, 29)] * pool
    elif config == 3:
        tv = rng.choice([t for t, _ in MIX_3], size=pool, p=[p for _, p in MIX_3])
        ptypes = [(int(t),) * 3 for t in tv]
    else:
        ptypes = [(GATE_T, GATE_T, DOWN_T)] * pool
    k = 1 if config == 0 else K
    lim = REAL_LIM if config == 6 else 0.0   # the SwiGLU limit the GPU layer uses
    mats = [orc.gen_expert(ptypes[e], SEED, 0, e, DIM, FF) for e in range(pool)]   # not timed
    draws = [(rng.choice(pool, size=k, replace=False).astype(np.int32), rng.random(k).astype(np.float32),
              rng.standard_normal(DIM).astype(np.float32)) for _ in range(64)]
    avx2 = orc.lane_avx2()

    def run(n_threads, seconds, min_reps=5):
        """2 warm-up layers, then layers until `seconds` (at least min_reps)."""
        times, phases, nbytes = [], np.zeros(5, np.float64), 0
        for i in range(2):
            ids, w, x = draws[i]
            orc.lane_layer([ptypes[e] for e in ids], [mats[e] for e in ids], ids, w, x, DIM, FF, threads=n_threads,
                           limit=lim)
        t_end = time.perf_counter() + seconds
        i = 0
        while len(times) < min_reps or time.perf_counter() < t_end:
            ids, w, x = draws[(2 + i) % len(draws)]
            i += 1
            t0 = time.perf_counter()
            orc.lane_layer([ptypes[e] for e in ids], [mats[e] for e in ids], ids, w, x, DIM, FF, threads=n_threads,
                           limit=lim, phases=phases)
            times.append(time.perf_counter() - t0)
            nbytes += sum(expert_bytes(ptypes[e]) for e in ids) + 2 * DIM * 4
        t = np.array(times)
        return {"us_per_layer": round(float(np.median(t)) * 1e6, 1), "us_min": round(float(t.min()) * 1e6, 1),
                "us_max": round(float(t.max()) * 1e6, 1), "layers": len(t),
                "GB_s": round(nbytes / t.sum() / 1e9, 3),
                "phases_us": dict(zip(("q1", "gate_up", "q2", "down", "combine"),
                                      (phases / len(t) / 1e3).round(1).tolist()))}

    per = {}
    if avx2:
        for n in workers:
            per[str(n)] = run(n, budget_s * (0.35 if n == 1 else 0.5 / max(1, len(workers) - 1)))
    best = str(workers[-1])
    # The reference's own scalar chain (q8k_core.hpp compiled from /root/reference), a few layers
    scalar = None
    if Reference.available():
        ref = Reference()
        t_all, nb, n_l = 0.0, 0, 0
        t_end = time.perf_counter() + budget_s * 0.15
        while n_l < 2 or time.perf_counter() < t_end:
            ids, w, x = draws[n_l % len(draws)]
            t0 = time.perf_counter()
            rows = np.stack([ref.expert(ptypes[e], *mats[e], DIM, FF, x, threads=share, limit=lim) for e in ids])
            ref.combine(ids, w, rows, np.zeros(DIM, np.float32))
            t_all += time.perf_counter() - t0
            nb += sum(expert_bytes(ptypes[e]) for e in ids) + 2 * DIM * 4
            n_l += 1
        scalar = {"kind": "reference", "GB_s": round(nb / t_all / 1e9, 3), "us_per_layer": round(t_all / n_l * 1e6, 1),
                  "threads": share, "layers": n_l,
                  "what": "the reference's own scalar q8k_core.hpp chain (oracle/_ref), 64-row jobs"}
    if not avx2:   # no AVX2 on this host: the scalar reference chain is the baseline
        return {"value": scalar["GB_s"] if scalar else None, "unit": "GB/s", "cores": share,
                "kind": "reference", "host": host, "sample": "host without AVX2: scalar reference chain only",
                "scalar_reference": scalar}
    top = per[best]
    return {
        "value": top["GB_s"], "unit": "GB/s", "cores": int(best), "kind": "port",
        "us_per_layer": top["us_per_layer"], "us_min": top["us_min"], "us_max": top["us_max"],
        "phases_us": top["phases_us"],
        "sample": f"{top['layers']} config-{config} layers ({k} expert(s) + combine each, drawn from {pool} generated "
                  f"experts) on the AVX2 restatement of the reference CPU lane (oracle/cpu_lane.c, bit-identical to "
                  f"the scalar restatement), {best} workers in 64-row jobs (the box's CPU share; physical cores "
                  f"{host['physical_cores']}, logical {host['logical_cpus']}), median of the timed layers",
        "workers": per,
        "host": dict(host, isa_used="AVX2 + FMA (256-bit)", box_share=share,
                     compiler="gcc -O2 -mfma -mavx2 -fopenmp -ffp-contract=off -fno-fast-math"),
        "scalar_reference": scalar,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0, help="timed steps (default: 2000 layers' worth)")
    ap.add_argument("--warmup", type=int, default=-1)
    ap.add_argument("--config", type=int, default=1, choices=(0, 1, 2, 3, 4, 5, 6))
    ap.add_argument("--tokens", type=int, default=512, help="config 4: tokens per grouped call")
    ap.add_argument("--device-route", action="store_true",
                    help="configs 1, 4: route each step on the GPU from N(0,1) logits (route.cpp router: "
                         "sqrt-softplus scores, top-6, normalized weights) inside the timed region")
    ap.add_argument("--per32", action="store_true",
                    help="configs 0-2: the per32 mode (the reference's production HIP lane arithmetic) "
                         "instead of the Q8_K chain")
    ap.add_argument("--routes", type=int, default=512)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    ap.add_argument("--cpu-threads", type=int, default=0, help="CPU baseline worker cap (default: the box's share)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true",
                    help="enqueue the timed steps onto a running stream (no device-side hold first)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "the routed-expert path runs on a single MI355X holding the whole bank", file=sys.stderr)
        sys.exit(2)
    cfg = args.config
    global DIM, FF
    if cfg == 6:   # the real expert shape; the rest of config 1's workload unchanged
        DIM, FF = REAL_DIM, REAL_FF
    if args.per32 and (cfg > 2 or args.device_route):
        print("bench.py: --per32 applies to configs 0-2 without --device-route", file=sys.stderr)
        sys.exit(2)
    L = N_LAYERS_3 if cfg == 3 else 1
    TOK = args.tokens if cfg == 4 else 1
    steps = args.steps or {3: 50, 4: 50}.get(cfg, 2000)
    warmup = args.warmup if args.warmup >= 0 else {3: 5, 4: 5}.get(cfg, 100)

    import torch
    import crosslane_amd as xl

    # ---- bank and routes
    if cfg == 3:
        types = mixed_types(L, SEED + 3)
    else:
        types = np.zeros((1, E, 3), np.int32)
        t3 = (29, 29, 29) if cfg == 2 else (GATE_T, GATE_T, DOWN_T)
        types[..., 0], types[..., 1], types[..., 2] = t3
    lane = xl.Lane(DIM, FF, L, E, types, max_picks=8, max_tokens=TOK if cfg == 4 else 0,
                   swiglu_limit=REAL_LIM if cfg == 6 else 0.0)
    lane.generate(SEED)
    n_r = args.routes
    if cfg == 0:
        rng = np.random.default_rng(SEED)
        ids = rng.integers(0, E, size=(n_r, 1, 1)).astype(np.int32)
        w = np.ones((n_r, 1, 1), np.float32)
        x = rng.standard_normal((n_r, DIM)).astype(np.float32)
    elif cfg == 2:
        ids, w, x = zipf_routes(n_r, SEED)
        ids, w = ids[:, None, :], w[:, None, :]
    elif cfg == 4:
        n_r = min(n_r, 8)   # route sets of TOK tokens each
        per = [routes(TOK, SEED + 200 + r) for r in range(n_r)]
        ids = np.stack([p[0] for p in per])   # [n_r, TOK, K]
        w = np.stack([p[1] for p in per])
        x = np.stack([p[2] for p in per])     # [n_r, TOK, DIM]
    elif cfg == 3:
        n_r = min(n_r, 64)
        per = [routes(n_r, SEED + 100 + l) for l in range(L)]
        ids = np.stack([p[0] for p in per], axis=1)
        w = np.stack([p[1] for p in per], axis=1)
        x = per[0][2]
    else:
        ids, w, x = routes(n_r, SEED)
        ids, w = ids[:, None, :], w[:, None, :]
    k = ids.shape[2]
    blk = None
    if cfg == 5:   # the MoE block around the layer: shared FFN, hc_post inputs
        srng = np.random.default_rng(SEED + 5)
        blk = {"mats": [dense_matrix(SHARED_T[0], FF, DIM, srng), dense_matrix(SHARED_T[1], FF, DIM, srng),
                        dense_matrix(SHARED_T[2], DIM, FF, srng)],
               "res": srng.standard_normal((n_r, HC_H, DIM)).astype(np.float32),
               "post": (srng.random((n_r, 8)) * 2).astype(np.float32),
               "comb": srng.random((n_r, 64)).astype(np.float32)}
    droute = args.device_route and cfg in (1, 4)
    if droute:   # fresh N(0,1) logits per route; the ids / weights come from the device router
        lrng = np.random.default_rng(SEED + 7)
        logits = lrng.standard_normal((n_r, TOK if cfg == 4 else 1, E)).astype(np.float32)
        from oracle.oracle import Oracle   # checker only: the expected picks for the byte count
        orc_ids = np.stack([Oracle().route(logits[r], K)[0] for r in range(n_r)])
        ids = orc_ids if cfg == 4 else orc_ids.reshape(n_r, 1, K)
    # algorithmic bytes per step, averaged over the routes the timed steps use
    used = [(warmup + i) % n_r for i in range(steps)]
    if cfg == 4:   # every touched expert once, plus the tokens in and out
        step_bytes = np.array([sum(expert_bytes(types[0, e]) for e in np.unique(ids[r])) + TOK * 2 * DIM * 4
                               for r in range(n_r)], np.float64)
    else:
        step_bytes = np.array([sum(expert_bytes(types[l, e]) for l in range(L) for e in ids[r, l]) + L * 2 * DIM * 4
                               for r in range(n_r)], np.float64)
    if cfg == 5:
        step_bytes += block_extra_bytes()
    bytes_per_step = float(step_bytes[used].mean())

    # A dedicated (non-default) stream: the library launches on it and the
    # timing events are recorded on it.
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    with torch.cuda.stream(stream):
        d_ids = torch.from_numpy(ids).cuda()
        d_w = torch.from_numpy(w).cuda()
        d_x = torch.from_numpy(x).cuda()
        d_h = torch.zeros((L + 1, DIM), dtype=torch.float32, device="cuda")   # config 3: final hiddens of the passes
        d_hn = torch.zeros(DIM, dtype=torch.float32, device="cuda")           # config 3: the carried hidden
        d_mix1 = torch.zeros(8, dtype=torch.float32, device="cuda")
        d_mix1[0] = 1.0
        d_ones = torch.ones(DIM, dtype=torch.float32, device="cuda")
        d_y = torch.zeros(DIM, dtype=torch.float32, device="cuda")             # config 3: layer outputs, alternating
        d_y2 = torch.zeros(DIM, dtype=torch.float32, device="cuda")
        d_out = torch.zeros((n_r, TOK, DIM) if cfg == 4 else (n_r, DIM), dtype=torch.float32, device="cuda")
        d_logits = torch.from_numpy(logits).cuda() if droute else None
        d_y32 = torch.zeros((K, DIM), dtype=torch.float32, device="cuda") if args.per32 else None
        if blk:
            d_mats = [torch.from_numpy(m).cuda() for m in blk["mats"]]
            d_res, d_post, d_comb = (torch.from_numpy(blk[key]).cuda() for key in ("res", "post", "comb"))
            d_h2 = torch.zeros((HC_H, DIM), dtype=torch.float32, device="cuda")
            d_work = torch.empty(xl.shared_work_bytes(DIM, FF, 1), dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()

    def step(i):
        r = i % n_r
        if droute and cfg == 4:
            lane.grouped_forward_routed_async(0, d_logits[r], K, d_x[r], d_out[r], stream=sp)
            return
        if droute:
            lane.layer_forward_routed_async(0, d_logits[r, 0], K, d_x[r], d_out[r], stream=sp)
            return
        if cfg == 4:
            lane.grouped_forward_async(0, d_ids[r], d_w[r], d_x[r], d_out[r], stream=sp)
            return
        if cfg == 5:   # the MoE block: routed layer, shared FFN added last, hc_post of the sum (one call)
            lane.moe_block_async(0, d_ids[r, 0], d_w[r, 0], d_x[r], SHARED_T, *d_mats, FF, d_work, d_res[r],
                                 d_post[r], d_comb[r], d_out[r], d_h2, stream=sp)
            return
        if args.per32:
            lane.layer_forward_per32_async(0, d_ids[r, 0], d_x[r], d_y32, w=d_w[r, 0], out=d_out[r], stream=sp)
            return
        if cfg != 3:
            lane.layer_forward_async(0, d_ids[r, 0], d_w[r, 0], d_x[r], d_out[r], stream=sp)
            return
        with torch.cuda.stream(stream):
            # layer l > 0 takes the RMS-normalized output of layer l - 1 (one stream,
            # mix 1, unit weight) inside its own launch; outputs alternate buffers
            ys = (d_y, d_y2)
            lane.layer_forward_async(0, d_ids[r, 0], d_w[r, 0], d_x[r], ys[0], stream=sp)
            for l in range(1, L):
                lane.layer_forward_prenorm_async(l, d_ids[r, l], d_w[r, l], ys[(l - 1) & 1].view(1, DIM), d_mix1,
                                                 d_ones, d_hn, ys[l & 1], eps=1e-6, stream=sp)
            lane.hc_pre_norm_async(ys[(L - 1) & 1].view(1, 1, DIM), d_mix1, d_ones, d_hn.view(1, DIM), eps=1e-6,
                                   stream=sp)
            d_h[r % (L + 1)].copy_(d_hn)   # the pass's final hidden (checked for finiteness after timing)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    # The stream is held by a short device-side sleep while the first timed
    # steps are enqueued, so that the first launch's host-side latency stays out
    # of the events' span (it weighs on short runs); the sleep ends before t0.
    hold_ms = 0.0
    if not args.no_prefill:
        h0 = torch.cuda.Event(enable_timing=True)
        h0.record(stream)
        with torch.cuda.stream(stream):
            torch.cuda._sleep(int(1e5))   # ~0.9 ms measured (the value is the spin kernel's clock ticks)
    t0.record(stream)
    wall0 = time.perf_counter()
    for i in range(steps):
        step(warmup + i)
    t1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    if not args.no_prefill:
        hold_ms = h0.elapsed_time(t0)
    lane.sync(sp)
    if cfg == 3:
        assert bool(torch.isfinite(d_h).all()), "non-finite hidden in the 40-layer pass"
    ms = t0.elapsed_time(t1)
    us_step = ms * 1e3 / steps
    us_layer = us_step / L   # config 4: one grouped call of TOK tokens
    gbs = bytes_per_step / (us_step * 1e-6) / 1e9

    # The spread, after the timed region: 20 batches of up to 25 further steps
    # (fresh routes as before), each batch between two events of its own,
    # enqueued behind a device-side sleep so that they run back to back rather
    # than at the host's enqueue pace (an event pair around every single step
    # would add its packets' cost to each step: +4.7 us at config 1)
    per_b = max(10, min(25, steps // 20))   # (a one-step batch would time mostly its events)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(20)]
    with torch.cuda.stream(stream):
        torch.cuda._sleep(int(5e7))   # ~25 ms at the shader clock: longer than enqueueing the batches
    i = warmup + steps
    for ea, eb in evs:
        ea.record(stream)
        for _ in range(per_b):
            step(i)
            i += 1
        eb.record(stream)
    torch.cuda.synchronize()
    lane.sync(sp)
    per = np.array([ea.elapsed_time(eb) * 1e3 / (per_b * L) for ea, eb in evs])
    dist = {"median": round(float(np.median(per)), 3), "p10": round(float(np.percentile(per, 10)), 3),
            "p90": round(float(np.percentile(per, 90)), 3), "batches": len(evs), "steps_per_batch": per_b,
            "how": "us per layer: mean of each batch of steps run back to back after the timed region, "
                   "each batch between its own events (whose packets add to the batch's time: the "
                   "median sits ~1 us above the timed region's figure at config 1)"}

    # One kernel launch per layer: the layer kernel's average duration is the
    # timed region's event time over the launches (rocprofv3 --kernel-trace of
    # the same command agrees; see profiles/). Config 3's figure also holds the
    # normalization inside the layer launches and the one after the last layer,
    # so it bounds the kernel from below.
    kernel = {0: "xl::dev::stream_kernel (single-launch layer, IQ2 instance)",
              1: "xl::dev::stream_kernel (single-launch layer, IQ2 instance)",
              2: "xl::dev::stream_kernel (single-launch layer, IQ1_M instance)",
              3: "xl::dev::stream_kernel (single-launch layer, mixed-type instance)",
              4: "grouped path (bucket, Q8_K, gu_kernel, Q8_K, dn_kernel, combine: 6 launches per step)"}.get(cfg)
    if cfg == 6:   # whichever single launch served the calls (xl_debug_launch_counts)
        counts = lane.launch_counts()
        kernel = ("xl::dev::stream_kernel (single-launch layer, IQ2 instance, 5120 x 2304)" if counts["stream"]
                  else "xl::dev::layer3_kernel (all-types single-launch layer)" if counts["alltypes"]
                  else "separate launches")
    if cfg == 5:
        kernel = ("MoE block (xl_moe_block_async): stream_kernel (routed layer; x quantized per 32 in its "
                  "prologue), mv32 shared gate+up, swiglu_quant32, mv32 shared down (+ the routed row, hc_post in "
                  "its epilogue): 4 launches per step")
    if args.per32:
        kernel = ("per32 chain (quant32, mv32 gate+up, swiglu_quant32, mv32 down with the fixed-order combine in its "
                  "epilogue: 4 launches per step)")
    traffic = measured_traffic() if cfg == 1 and not args.per32 else None

    cpu = None
    if not args.no_cpu and not args.per32 and cfg != 5:   # the CPU baseline times the Q8_K chain
        cpu = cpu_baseline(args.cpu_seconds, config=1 if cfg == 4 else cfg, max_threads=args.cpu_threads)
        if cfg == 4 and cpu["value"] is not None:   # the CPU lane has no grouping: TOK per-token layers per step
            cpu["value"] = round(bytes_per_step / (cpu["us_per_layer"] * 1e-6 * TOK) / 1e9, 3)
            cpu["sample"] += f"; per step = {TOK} such token layers (algorithmic bytes of the grouped step)"

    workloads = {
        0: "config0: one expert per step (k=1, w=1) of 384 resident, d_model 4096, d_ff 3072, "
           "gate/up IQ2_XXS + down IQ2_XS",
        1: "config1: MoE layer, decode batch 1, top-6 of 384 resident experts, d_model 4096, "
           "d_ff 3072, gate/up IQ2_XXS + down IQ2_XS, fixed-order combine",
        2: "config2: MoE layer, decode batch 1, all-IQ1_M bank of 384, 6 distinct experts ~ rank^-1.1 (Zipf), "
           "fixed-order combine",
        3: "config3: 40-layer pass per token, 40 x 384 experts typed 17% IQ2_XS / 19% IQ2_XXS / 64% IQ1_M, "
           "top-6 per layer, hidden carried through RMS normalization",
        4: f"config4: grouped, {TOK} tokens x N(0,1)[4096], per-token top-6 of 384 config-1 experts, "
           "fixed-order combine per token",
        5: "config5: MoE block of one token: shared-expert FFN (Q5_K gate/up, Q6_K down, 4096x3072, per32), "
           "config-1 routed layer with the shared row added last, hc_post over 4 streams",
        6: "config6: config 1 at the real expert shape, d_model 5120, d_ff 2304, SwiGLU limit 10, top-6 of 384 "
           "resident experts, gate/up IQ2_XXS + down IQ2_XS, fixed-order combine",
    }
    line = {
        "metric": "routed-expert µs/layer (top-6, batch 1) + achieved HBM GB/s vs MI355X peak",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms / steps, 6), "us_per_layer": round(us_layer, 3),
        "us_per_layer_dist": dist,
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic (seeded IQ blocks generated on device, N(0,1) activations and router logits)",
        "config": {"workload": workloads[cfg] + ("; routed on the GPU each step (route.cpp router)" if droute else "")
                    + ("; per32 mode (per-32 int8 activations, hip_experts.hip arithmetic)" if args.per32 else ""),
                   "layers_per_step": L, "tokens_per_step": TOK,
                   "bytes_per_step": int(round(bytes_per_step)), "routes": n_r},
        "roofline": {"bound": "hbm", "kernel": kernel,
                     "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": int(round(bytes_per_step / L)), "us_per_launch": round(us_layer, 3)},
        "cpu_baseline": cpu,
        "host_wall_us_per_step": round(wall * 1e6 / steps, 3),
        "timing": ("the first timed steps enqueued behind a %.2f ms device-side hold" % hold_ms)
                  if not args.no_prefill else "timed steps enqueued onto the running stream",
    }
    print(json.dumps(line), flush=True)
    lane.close()


if __name__ == "__main__":
    main()
