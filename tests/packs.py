"""Writes small weight packs in the reference's layout for the loader tests:
ds4.txt + tensors.txt over shard files, routed experts named
layers.<l>.ffn.experts.<e>.w1 / w3 / w2 .weight (gate / up / down) holding raw
ggml blocks (the layout of engine/strata/sycl/stage/wiring/pack_source.cpp:
144-186; engine/strata/warm/test_mmvq.py:111-137 builds packs the same way).
The blocks come from the oracle's seeded generator (seed, layer, expert, role),
so a test can recompute any matrix."""
from __future__ import annotations

import os

NAMES = {16: "IQ2_XXS", 17: "IQ2_XS", 29: "IQ1_M"}
ROLE = ("w1", "w3", "w2")


def write_pack(path, orc, sigs, dim, ff, n_experts, seed, shards=2, top_k=6, swiglu_limit=None):
    """sigs[l] = (gate, up, down) ggml types of layer l. Returns path."""
    os.makedirs(path, exist_ok=True)
    meta = {"model_dir": path, "format": "gguf", "hidden_size": dim, "num_hidden_layers": len(sigs),
            "n_routed_experts": n_experts, "num_experts_per_tok": top_k, "moe_intermediate_size": ff}
    if swiglu_limit is not None:
        meta["swiglu_limit"] = swiglu_limit
    with open(os.path.join(path, "ds4.txt"), "w") as f:
        f.write("".join(f"{k} {v}\n" for k, v in meta.items()))
    data = [bytearray() for _ in range(shards)]
    lines = [f"file {i} shard{i}.gguf" for i in range(shards)]
    for l, sig in enumerate(sigs):
        for e in range(n_experts):
            for r, t in enumerate(sig):
                n, k = (ff, dim) if r < 2 else (dim, ff)
                raw = orc.gen_matrix(t, seed, l, e, r, n, k).tobytes()
                sh = (l + e + r) % shards
                lines.append(f"t layers.{l}.ffn.experts.{e}.{ROLE[r]}.weight {NAMES[t]} {sh} {len(data[sh])} {len(raw)} "
                             f"{k} {n}")
                data[sh].extend(raw)
    for i in range(shards):
        with open(os.path.join(path, f"shard{i}.gguf"), "wb") as f:
            f.write(data[i])
    with open(os.path.join(path, "tensors.txt"), "w") as f:
        f.write("\n".join(lines) + "\n")
    return path
