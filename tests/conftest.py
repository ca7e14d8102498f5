"""Shared test setup: the `gpu` marker, paths, and the parity metric."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


# Parity bar for floating-point outputs (north_star: logits within 1e-9 max
# relative error).  The denominator is floored at 1e-3 of the array's RMS so
# that entries which happen to sit near zero are judged on the array's scale.
REL_TOL = 1e-9


def max_rel_err(got, want) -> float:
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (got.shape, want.shape)
    scale = np.sqrt(np.mean(np.abs(want) ** 2)) if want.size else 0.0
    den = np.maximum(np.abs(want), 1e-3 * scale)
    den = np.where(den == 0, 1.0, den)
    return float(np.max(np.abs(got - want) / den)) if want.size else 0.0


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    oracle.lib()
    return oracle
