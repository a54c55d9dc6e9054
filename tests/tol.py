"""Parity tolerance of the HIP path against the CPU reference GDN.

fp32 kernels: |gpu - ref| <= ATOL + RTOL * |ref| elementwise on outputs and
final state (max-abs 2e-3 / rel 1e-3).
"""
import numpy as np

ATOL = 2e-3
RTOL = 1e-3


def assert_close(gpu, ref, atol=ATOL, rtol=RTOL, what=""):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    assert gpu.shape == ref.shape, (what, gpu.shape, ref.shape)
    err = np.abs(gpu - ref)
    bad = err > atol + rtol * np.abs(ref)
    if bad.any():
        i = np.unravel_index(np.argmax(err - (atol + rtol * np.abs(ref))), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} of {bad.size} outside tolerance; worst at {i}: "
                             f"gpu={gpu[i]:.6g} ref={ref[i]:.6g} (max abs err {err.max():.3g})")
    return float(err.max())
