import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


def rand_events(n=500, B=2, H=20, W=24, seed=0):
    """Random events in [-2, W+2) x [-2, H+2), weights in [0.1, 1.1), sorted by (b, t); the shape of the
    reference's test inputs (tests/test_ops.py:16-23), drawn with NumPy."""
    rng = np.random.default_rng(seed)
    pos = np.stack([rng.random(n) * (W + 4) - 2, rng.random(n) * (H + 4) - 2], 1).astype(np.float32)
    w = (rng.random(n) + 0.1).astype(np.float32)
    b = rng.integers(0, B, n).astype(np.int64)
    t = rng.random(n).astype(np.float32)
    order = np.argsort(b.astype(np.float64) * 4 + t.astype(np.float64), kind="stable")
    return pos[order], w[order], b[order], t[order]


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


def assert_sums_close(got, want, rel=1e-5):
    """Per-anchor relative bar for pair sums: a sum of positive kernel terms, each at least exp(-cut^2 / 2), so
    every anchor is held to |got - want| <= rel * want; anchors without a contributing pair read exactly 0."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    assert g.shape == w.shape
    zero = w == 0
    assert np.all(g[zero] == 0), f"{int((g[zero] != 0).sum())} anchors without pairs read non-zero"
    err = np.abs(g - w)
    bad = err > rel * w
    worst = float((err[~zero] / w[~zero]).max()) if (~zero).any() else 0.0
    assert not bad.any(), f"{int(bad.sum())} of {w.size} sums off by more than {rel:g} relative (worst {worst:.2e})"


def assert_logs_close(got, want, tol=1e-5):
    """Log predictive densities: |got - want| <= tol per anchor, i.e. the densities themselves within tol
    relative."""
    err = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    assert float(err.max(initial=0.0)) <= tol, f"{int((err > tol).sum())} log scores off by more than {tol:g} " \
                                               f"(worst {float(err.max()):.2e})"
