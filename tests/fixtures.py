"""Load the golden GDN fixtures and regenerate their inputs (hash-checked)."""
from __future__ import annotations

import hashlib
import os

import numpy as np

from overhang_amd import synth
from overhang_amd.dims import GdnDims

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LAYER_FIXTURES = ["cfg1_layer_f32", "tiny_layer_int8"]
CORE_FIXTURES = ["core_rep3_d16", "core_kd32_vd16", "core_d128", "core_d32_decay"]


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def load(name: str):
    """Returns (dims, weights, inputs, initial (conv, S), expected dict)."""
    f = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    kh, vh, kd, vd, K, hidden = (int(v) for v in f["dims"])
    d = GdnDims(kh, vh, kd, vd, K, hidden, float(f["eps"]))
    seed, T = int(f["seed"]), int(f["T"])
    kind = str(f["kind"])
    if kind == "layer":
        w = synth.layer_weights(d, seed, gnorm_std=float(f["gnorm_std"]))
        inp = {"x": synth.normal(seed, synth.S_X, (T, d.hidden))}
        if int(f["zero_state"]):
            conv = np.zeros((d.conv_dim, d.K - 1), np.float32)
            S = np.zeros((d.vh, d.kd, d.vd), np.float32)
        else:
            conv, S = synth.states(d, seed)
        exp = {"out": f["out"], "conv": f["conv"], "S": f["S"], "int8": bool(int(f["int8"]))}
    else:
        w = synth.layer_weights(d, seed, gnorm_std=float(f["gnorm_std"]), projections=False)
        inp = synth.core_inputs(d, T, seed, a_mean=float(f["a_mean"]))
        conv, S = synth.states(d, seed)
        exp = {"core": f["core"], "conv": f["conv"], "S": f["S"]}
    for k, v in list(w.items()) + list(inp.items()):
        assert sha(v) == str(f["sha_" + k]), f"{name}: regenerated input {k} differs from the fixture's"
    assert sha(conv) == str(f["sha_conv0"]) and sha(S) == str(f["sha_S0"])
    return d, w, inp, (conv, S), exp
