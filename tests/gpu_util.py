"""Shared helpers of the GPU parity tests.

fp32 tolerance: "1e-4 relative" is read per row (one logits / activation
vector), normwise: max_i |a_i - b_i| / max_i |b_i| <= 1e-4.  An elementwise
ratio is not usable for vectors whose entries cross zero: two correct fp32
dot products of length 4096 summed in different orders differ by ~4e-6 of
the row scale, which is an unbounded relative error on entries near zero.
Where an exact value is cheap (float64), the tests also require the device
error to be no larger than a small multiple of the oracle's own fp32 error.
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "neural-network_amd", "python"))

import nnhip  # noqa: E402


def row_rel_err(a, b):
    """max over rows of max|a - b| / max|b| (normwise relative error)."""
    a = np.asarray(a, np.float64).reshape(-1, np.shape(a)[-1])
    b = np.asarray(b, np.float64).reshape(-1, np.shape(b)[-1])
    scale = np.maximum(np.abs(b).max(axis=1), 1e-30)
    return float((np.abs(a - b).max(axis=1) / scale).max())


def assert_rows_close(a, b, tol=1e-4, what=""):
    e = row_rel_err(a, b)
    assert e <= tol, f"{what}: max row-relative error {e:.3g} > {tol}"
    return e


def assert_as_accurate(dev, oracle, exact, factor=4.0, what=""):
    """The device result is within `factor` times the oracle's own distance
    from the exact (float64) result, row by row (plus 1e-7 of the row
    scale for rows the oracle gets nearly exact)."""
    dev = np.asarray(dev, np.float64).reshape(-1, np.shape(dev)[-1])
    orc = np.asarray(oracle, np.float64).reshape(-1, np.shape(oracle)[-1])
    ex = np.asarray(exact, np.float64).reshape(-1, np.shape(exact)[-1])
    scale = np.abs(ex).max(axis=1)
    e_dev = np.abs(dev - ex).max(axis=1)
    e_orc = np.abs(orc - ex).max(axis=1)
    bad = e_dev > factor * e_orc + 1e-7 * scale
    assert not bad.any(), (f"{what}: device error {e_dev[bad][:3]} vs oracle "
                           f"{e_orc[bad][:3]}")
