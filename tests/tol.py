"""Parity tolerance of the HIP path against the CPU reference GDN.

fp32 kernels: |gpu - ref| <= ATOL + RTOL * |ref| elementwise on outputs and
final state (max-abs 2e-3 / rel 1e-3).

Every comparison records its margin: the largest absolute error and the
largest ratio err / (ATOL + RTOL*|ref|) (1.0 = at the bound).  The test
session prints them per test at its end (tests/conftest.py).
"""
import os

import numpy as np

ATOL = 2e-3
RTOL = 1e-3

# (test node id, what, max abs err, max rel err, worst err/bound ratio)
MARGINS = []


def _current_test() -> str:
    return os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0]


def assert_close(gpu, ref, atol=ATOL, rtol=RTOL, what=""):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    assert gpu.shape == ref.shape, (what, gpu.shape, ref.shape)
    err = np.abs(gpu - ref)
    bound = atol + rtol * np.abs(ref)
    ratio = err / bound
    mx = float(err.max()) if err.size else 0.0
    rel = float((err / np.maximum(np.abs(ref), 1e-30)).max()) if err.size else 0.0
    worst = float(ratio.max()) if err.size else 0.0
    MARGINS.append((_current_test(), what, mx, rel, worst))
    bad = ratio > 1.0
    if bad.any():
        i = np.unravel_index(np.argmax(ratio), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tolerance; worst at {i}: "
                             f"gpu={gpu[i]:.6g} ref={ref[i]:.6g} (max abs err {mx:.3g})")
    return mx
