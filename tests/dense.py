"""Seeded dense-format matrices (the shared-expert formats Q8_0, Q4_K, Q5_K,
Q6_K) for tests: uniform random bytes with every fp16 scale field set to a
finite value in [1e-3, 1e-2), rows of k / (values per block) ggml blocks."""
from __future__ import annotations

import numpy as np

DENSE_BYTES = {8: 34, 12: 144, 13: 176, 14: 210}
DENSE_VALUES = {8: 32, 12: 256, 13: 256, 14: 256}
DENSE_NAMES = {8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K"}


def _half_scales(rng, n):
    return rng.uniform(1e-3, 1e-2, n).astype(np.float16).view(np.uint16)


def dense_matrix(t: int, n: int, k: int, seed: int) -> np.ndarray:
    """n x k matrix of type t as raw ggml bytes (uint8, n * row bytes)."""
    rng = np.random.default_rng(seed * 131 + t)
    nb = n * (k // DENSE_VALUES[t])
    blocks = rng.integers(0, 256, size=(nb, DENSE_BYTES[t]), dtype=np.uint8)
    fields = {8: (0,), 12: (0, 2), 13: (0, 2), 14: (208,)}[t]
    for off in fields:
        blocks[:, off:off + 2] = _half_scales(rng, nb).view(np.uint8).reshape(nb, 2)
    return blocks.reshape(-1)
