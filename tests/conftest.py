"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on CPU."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle.oracle import Oracle, Reference  # noqa: E402  (test infrastructure)

REFERENCE_TREE = "/root/reference/engine/strata"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu)")


@pytest.fixture(scope="session")
def orc() -> Oracle:
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    if not Reference.available():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    return Reference()


@pytest.fixture
def rng():
    return np.random.default_rng(20261201)


def max_rel(a: np.ndarray, b: np.ndarray) -> float:
    """Max-norm relative error ||a - b||_inf / ||b||_inf (0 for b == a == 0)."""
    a = np.asarray(a, dtype=np.float64); b = np.asarray(b, dtype=np.float64)
    den = np.max(np.abs(b))
    num = np.max(np.abs(a - b))
    return 0.0 if num == 0 else float(num / den) if den > 0 else float("inf")
