import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and librxw8.so")


def golden_npz(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def golden_json(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def rel_err(actual, expected):
    """Normwise relative error: max|a - e| / max|e| (the parity metric)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    den = np.max(np.abs(e))
    return float(np.max(np.abs(a - e)) / (den if den > 0 else 1.0))


def elem_rel_err(actual, expected, floor=1e-2):
    """Per-element relative error: max_i |a_i - e_i| / max(|e_i|, floor * rms(e)).
    Unlike the normwise metric it sees a corrupted small output; the floor
    keeps outputs that cancel to ~0 from dividing by ~0."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    rms = float(np.sqrt(np.mean(e * e))) if e.size else 0.0
    den = np.maximum(np.abs(e), floor * rms if rms > 0 else 1.0)
    return float(np.max(np.abs(a - e) / den)) if e.size else 0.0


@pytest.fixture(scope="session")
def rt():
    """GPU runtime (only for tests marked gpu)."""
    import rxla_amd

    r = rxla_amd.Runtime(0)
    yield r
    r.synchronize()
