"""CPU-side checks of the C-ABI library: it loads, exports every entry point
include/om_hip.h declares, and reports a missing device instead of falling
back to anything.  Also pins the product's host-side int8 quantiser to the
reference rule (via the oracle)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import oracle
from overhang_amd import gdn, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "om_hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(omh_\w+)\s*\(", src)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(gdn.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = gdn.lib()
    for name in declared_symbols():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", gdn.LIB_PATH], capture_output=True, text=True).stdout
    for name in declared_symbols():
        assert re.search(rf"\bT {name}$", out, re.M), f"{name} not a defined text symbol"


def test_library_carries_gfx950_code_object():
    blob = open(gdn.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob


def test_init_without_device_fails_loudly():
    if gdn.lib().omh_init():
        pytest.skip("a device is present")
    assert "device" in gdn.last_error().lower() or "om_hip" in gdn.last_error().lower()
    w = synth.layer_weights(synth_dims(), 0, projections=False)
    with pytest.raises(gdn.OmhError):
        gdn.GdnLayer(0, synth_dims(), w)
    # raw entry points return the device error code rather than computing anything
    assert gdn.lib().omh_gdn_decode(0, 1, None, None) == gdn.OMH_ERR_DEVICE


def test_opt_out_env_is_honoured():
    code = ("import ctypes,sys; L=ctypes.CDLL(sys.argv[1]); "
            "L.omh_last_error.restype=ctypes.c_char_p; "
            "print(L.omh_init(), L.omh_last_error().decode())")
    r = subprocess.run(["python", "-c", code, gdn.LIB_PATH], capture_output=True, text=True,
                       env={**os.environ, "OM_HIP": "0"})
    assert r.stdout.startswith("0 ") and "OM_HIP=0" in r.stdout


def synth_dims():
    from overhang_amd.dims import CFG1
    return CFG1


def test_host_quantiser_matches_reference_rule():
    f = np.load(os.path.join(ROOT, "tests", "golden", "quant_rows.npz"), allow_pickle=False)
    q, s = gdn.quantize_rows(f["W"])
    assert np.array_equal(q, f["q"]) and np.array_equal(s, f["s"])
    W = synth.normal(3, 3, (64, 256), 0.0, 0.02)
    q1, s1 = gdn.quantize_rows(W)
    q2, s2 = oracle.quantize_rows(W)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)
