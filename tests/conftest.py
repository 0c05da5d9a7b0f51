"""Shared pytest configuration.

``-m "not gpu"`` runs the oracle-vs-golden tests, the host logic and the C-ABI
export checks; ``-m gpu`` runs the parity tests through the HIP library.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


def same(actual, expected, label=""):
    """Bit-identity check that reports cheaply on failure (a byte-string
    comparison would make pytest build a diff of the whole buffers)."""
    import numpy as np

    a = np.ascontiguousarray(actual)
    e = np.ascontiguousarray(expected).reshape(a.shape) if np.size(expected) == a.size else np.ascontiguousarray(expected)
    if a.shape != e.shape or a.dtype != e.dtype:
        raise AssertionError(f"{label}: shape/dtype {a.shape}/{a.dtype} vs {e.shape}/{e.dtype}")
    au = a.view(np.uint8).reshape(-1, a.dtype.itemsize) if a.size else a.view(np.uint8)
    eu = e.view(np.uint8).reshape(-1, e.dtype.itemsize) if e.size else e.view(np.uint8)
    if np.array_equal(au, eu):
        return
    bad = np.flatnonzero((au != eu).any(axis=-1))
    af, ef = a.ravel(), e.ravel()
    msg = f"{label}: {bad.size} of {a.size} elements differ; first at {bad[:5].tolist()}: " \
          f"got {af[bad[:5]].tolist()} want {ef[bad[:5]].tolist()}"
    if a.dtype.kind == "f":
        msg += f"; max |diff| {np.abs(af.astype(np.float64) - ef.astype(np.float64)).max():.6g}"
    raise AssertionError(msg)


def load_golden(name):
    import json

    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o

    o.build()
    return o
