"""Shared test setup: import paths, the ``gpu`` marker and fixture loaders."""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "callaghandev.ml_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def ops_golden():
    with np.load(os.path.join(GOLDEN, "ops.npz")) as z:
        return {k: z[k] for k in z.files}


def load_lm_golden(name: str):
    from cdml import synth

    with np.load(os.path.join(GOLDEN, f"{name}.npz")) as z:
        g = {k: z[k] for k in z.files}
    cfg = {str(k): int(v) for k, v in zip(g["cfg_keys"], g["cfg_vals"])}
    g["cfg"] = cfg
    g["weights"] = synth.lm_weights(cfg, int(g["seed"]), biased=True)
    return g


def assert_parity(actual, expected, atol=1e-4, rtol=1e-3, what=""):
    """The path's parity predicate: |a - e| <= atol + rtol |e| per element."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    assert np.all(np.isfinite(a)), f"{what}: non-finite values"
    err = np.abs(a - e)
    bad = err > atol + rtol * np.abs(e)
    if bad.any():
        i = np.unravel_index(np.argmax(err - (atol + rtol * np.abs(e))), e.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {e.size} elements out of tolerance "
            f"(atol {atol}, rtol {rtol}); worst at {i}: got {a[i]}, want {e[i]}; "
            f"max abs err {err.max():.3e}")


def assert_parity_with_exact(actual, oracle, exact, atol=1e-4, rtol=1e-3, what=""):
    """Parity for long fp32 reductions (weight gradients summed over thousands
    of rows).  The oracle sums in the reference's sequential fp32 order, and on
    elements that cancel to near zero its own rounding can exceed the bar: a
    2048-row gradient sum of O(1) products drifts by up to 3e-4 from exact
    arithmetic.  So the result must meet the bar against the float64 value
    everywhere, and against the oracle wherever the oracle is within half the
    bar of the float64 value.  (With the full bar as the selection, an
    element where the oracle is off by 0.9 of the bar fails even when the
    result is off by 0.15 of it in the other direction: a 4100-row sum
    measured exactly that.)"""
    e64 = np.asarray(exact, np.float64)
    o = np.asarray(oracle, np.float64)
    assert_parity(actual, e64, atol, rtol, what + " (vs float64)")
    ok = np.abs(o - e64) <= 0.5 * (atol + rtol * np.abs(e64))
    assert_parity(np.asarray(actual)[ok], o[ok], atol, rtol, what + " (vs oracle)")
