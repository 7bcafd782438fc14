"""CPU: the ggml codebooks in the product (crosslane_amd/csrc/xl_codebooks.inc,
2-bit symbols) and in the oracle (oracle/orc_codebooks.inc, base-3 rows) are
two independent encodings. Both must expand to the same u64 rows, whose
SHA-256 was taken from the reference's q8k_tables.inc (sycl/stage/wiring/
q8k_tables.inc:3,517,647,713); where the reference tree is present the text is
parsed and compared entry by entry."""
from __future__ import annotations

import hashlib
import os
import re

import numpy as np
import pytest

import crosslane_amd as xl
from tests.conftest import REFERENCE_TREE

SHA = {
    0: "05826b5d3e472a3a78f196be62ac78acf81df0f909626e12ab9fa2a5d490dd54",  # iq2xxs_grid[256]
    1: "06e47aaca60b4dc1d9b5a3f34540437058a6b142b4d7a59d5ded769b4d1bf1de",  # iq2xs_grid[512]
    2: "07540ffc1aeaf6ad4d97e96b0fcc765aae39671d4ae4a27bbd0e796fde167c6a",  # iq1s_grid[2048]
}
KSIGNS_SHA = "a76742a603f8beca5212ecce0f1f02f11a4887fd2f7c8b15aca0ea3eb3380c31"


def sha(rows: np.ndarray) -> str:
    return hashlib.sha256(rows.astype("<u8").tobytes()).hexdigest()


@pytest.mark.parametrize("which", [0, 1, 2])
def test_product_and_oracle_tables(orc, which):
    prod = xl.codebook(which)
    assert np.array_equal(prod, orc.codebook(which))
    assert sha(prod) == SHA[which]


def test_ksigns():
    ks = xl.codebook(3).astype(np.uint8)
    assert hashlib.sha256(ks.tobytes()).hexdigest() == KSIGNS_SHA


@pytest.mark.parametrize("which", [0, 1, 2, 3])
def test_tables_vs_reference_build(ref, which):
    assert np.array_equal(xl.codebook(which), ref.table(which))


@pytest.mark.skipif(not os.path.isdir(REFERENCE_TREE), reason="reference tree absent")
def test_tables_vs_reference_text():
    src = open(os.path.join(REFERENCE_TREE, "sycl/stage/wiring/q8k_tables.inc")).read()
    for which, name in ((0, "iq2xxs_grid"), (1, "iq2xs_grid"), (2, "iq1s_grid"), (3, "ksigns_iq2xs")):
        m = re.search(name + r"\[(\d+)\]\s*=\s*\{(.*?)\};", src, re.S)
        vals = np.array([int(v, 0) for v in re.findall(r"0x[0-9a-fA-F]+|\d+", m.group(2))], dtype=np.uint64)
        assert np.array_equal(xl.codebook(which), vals)
