#!/usr/bin/env python3
"""Write the golden GDN vectors from the reference engine's own code.

Runs in the build container only (it needs oracle/_ref, compiled from the
reference sources by oracle/Makefile).  Each fixture stores the outputs of the
reference deltanet_step (overhang engines/qwen.c:301-364) and the sha256 of
every input array; the inputs themselves are regenerated from
overhang_amd.synth by the tests, which first check the hashes.

Core-only fixtures drive the reference layer with selector projections:
hidden = conv_dim + vh*vd + 2*vh, x = [qkv | z | b | a], W_qkv/W_z/W_b/W_a
pick their slice (one-hot rows) and W_out = [I; 0], so every projection is
exact and out[:vh*vd] is the reference core output.

Also copies the reference's tiny end-to-end oracle (model, config, token ids).

usage: python tests/golden/make_golden.py [attn]
"""
from __future__ import annotations

import hashlib
import os
import shutil
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from overhang_amd import synth  # noqa: E402
from overhang_amd.dims import GdnDims, CFG1, TINY  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
REF = os.environ.get("REF", "/root/reference")


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def selector_weights(d: GdnDims, w: dict) -> tuple[GdnDims, dict]:
    cd, vd_, vh = d.conv_dim, d.val_dim, d.vh
    H = cd + vd_ + 2 * vh
    dd = GdnDims(d.kh, d.vh, d.kd, d.vd, d.K, H, d.eps)
    W_qkv = np.zeros((cd, H), np.float32); W_qkv[np.arange(cd), np.arange(cd)] = 1
    W_z = np.zeros((vd_, H), np.float32); W_z[np.arange(vd_), cd + np.arange(vd_)] = 1
    W_b = np.zeros((vh, H), np.float32); W_b[np.arange(vh), cd + vd_ + np.arange(vh)] = 1
    W_a = np.zeros((vh, H), np.float32); W_a[np.arange(vh), cd + vd_ + vh + np.arange(vh)] = 1
    W_out = np.zeros((H, vd_), np.float32); W_out[np.arange(vd_), np.arange(vd_)] = 1
    ww = dict(w)
    ww.update(W_qkv=W_qkv, W_z=W_z, W_b=W_b, W_a=W_a, W_out=W_out)
    return dd, ww


def layer_fixture(name, d, seed, T, int8, zero_state, gnorm_std):
    w = synth.layer_weights(d, seed, gnorm_std=gnorm_std)
    x = synth.normal(seed, synth.S_X, (T, d.hidden))
    if zero_state:
        conv = np.zeros((d.conv_dim, d.K - 1), np.float32)
        S = np.zeros((d.vh, d.kd, d.vd), np.float32)
    else:
        conv, S = synth.states(d, seed)
    out, conv2, S2 = oracle.ref_layer_seq(d, w, x, conv, S, int8=int8)
    meta = dict(kind="layer", dims=np.array([d.kh, d.vh, d.kd, d.vd, d.K, d.hidden]),
                eps=np.float64(d.eps), seed=seed, T=T, int8=int(int8),
                zero_state=int(zero_state), gnorm_std=np.float64(gnorm_std))
    hashes = {"sha_" + k: sha(v) for k, v in w.items()}
    hashes.update(sha_x=sha(x), sha_conv0=sha(conv), sha_S0=sha(S))
    np.savez_compressed(os.path.join(OUT, name + ".npz"), out=out, conv=conv2, S=S2,
                        **meta, **hashes)
    print(f"{name}: out max|.| {np.abs(out).max():.4g}  S max|.| {np.abs(S2).max():.4g}")


def core_fixture(name, d, seed, T, gnorm_std, a_mean=0.0):
    w = synth.layer_weights(d, seed, gnorm_std=gnorm_std, projections=False)
    inp = synth.core_inputs(d, T, seed, a_mean=a_mean)
    conv, S = synth.states(d, seed)
    dd, ww = selector_weights(d, w)
    x = np.concatenate([inp["qkv"], inp["z"], inp["b"], inp["a"]], axis=1)
    out, conv2, S2 = oracle.ref_layer_seq(dd, ww, x, conv, S)
    core = out[:, :d.val_dim].copy()
    meta = dict(kind="core", dims=np.array([d.kh, d.vh, d.kd, d.vd, d.K, 0]),
                eps=np.float64(d.eps), seed=seed, T=T, gnorm_std=np.float64(gnorm_std),
                a_mean=np.float64(a_mean))
    hashes = {"sha_" + k: sha(v) for k, v in list(w.items()) + list(inp.items())}
    hashes.update(sha_conv0=sha(conv), sha_S0=sha(S))
    np.savez_compressed(os.path.join(OUT, name + ".npz"), core=core, conv=conv2, S=S2,
                        **meta, **hashes)
    print(f"{name}: core max|.| {np.abs(core).max():.4g}  S max|.| {np.abs(S2).max():.4g}")


def quant_fixture(name):
    rng_rows = synth.normal(7, 1, (6, 64), 0.0, 0.05)
    s_tie = np.float32(0.01)
    tie_row = (np.arange(64, dtype=np.float32) - 32 + 0.5) * s_tie      # .5 ties
    tie_row[0] = 127 * s_tie                                           # pins the scale
    W = np.concatenate([rng_rows,
                        np.zeros((1, 64), np.float32),                 # scale floor 1e-8
                        np.full((1, 64), 1e-12, np.float32),           # below the floor
                        tie_row[None, :]], axis=0).astype(np.float32)
    q, s = oracle.ref_quantize_rows(W)
    x = synth.normal(7, 2, (64,))
    y = oracle.ref_matmul_q(x, q, s)
    yf = oracle.ref_matvec(x, W)
    np.savez_compressed(os.path.join(OUT, name + ".npz"), W=W, x=x, q=q, s=s, y=y, yf=yf)
    print(f"{name}: scales {s}")


# (name, hidden, H, KV, hd, rot, pos0, T, int8, seed): the reference tiny
# model's attention shape (oracle/qwen_tiny/config.json: head_dim 32,
# partial_rotary_factor 0.25) and the Qwen3.6-35B-A3B one (hidden 2048, 16
# query / 2 kv heads of 256, rot 64), at positions below attn_step's
# float[8192] score buffer (qwen.c:407).
ATTN_FIXTURES = [
    ("attn_tiny_f32", 64, 4, 2, 32, 8, 1000, 3, False, 11),
    ("attn_tiny_int8", 64, 4, 2, 32, 8, 37, 4, True, 12),
    ("attn_35b_f32", 2048, 16, 2, 256, 64, 5000, 2, False, 13),
    ("attn_35b_int8", 2048, 16, 2, 256, 64, 8000, 3, True, 14),
]
ATTN_THETA, ATTN_EPS = 1e7, 1e-6


def attn_fixture(name, D, H, KV, hd, rot, pos0, T, int8, seed):
    w = synth.attn_weights(D, H, KV, hd, seed)
    x, Kpre, Vpre = synth.attn_inputs(D, KV, hd, pos0, T, seed)
    out, Kn, Vn = oracle.ref_attn_run(w, H, KV, hd, rot, ATTN_THETA, ATTN_EPS, pos0, Kpre, Vpre, x,
                                      int8=int8)
    meta = dict(kind="attn", dims=np.array([D, H, KV, hd, rot, pos0, T]), theta=np.float64(ATTN_THETA),
                eps=np.float64(ATTN_EPS), int8=int(int8), seed=seed)
    hashes = {"sha_" + k: sha(v) for k, v in w.items()}
    hashes.update(sha_x=sha(x), sha_Kpre=sha(Kpre), sha_Vpre=sha(Vpre))
    np.savez_compressed(os.path.join(OUT, name + ".npz"), out=out, K=Kn, V=Vn, **meta, **hashes)
    print(f"{name}: out max|.| {np.abs(out).max():.4g}")


def copy_tiny_model():
    dst = os.path.join(OUT, "qwen_tiny")
    os.makedirs(dst, exist_ok=True)
    for f in ("config.json", "generation_config.json", "model.safetensors"):
        shutil.copyfile(os.path.join(REF, "oracle", "qwen_tiny", f), os.path.join(dst, f))
    shutil.copyfile(os.path.join(REF, "oracle", "ref_qwen.json"), os.path.join(dst, "ref_qwen.json"))
    print("qwen_tiny copied")


def main():
    if oracle.ref_lib() is None:
        sys.exit("oracle/_ref/libqwen_ref.so missing: run `make -C oracle` with the reference present")
    if sys.argv[1:] == ["attn"]:                  # the attention fixtures alone
        for f in ATTN_FIXTURES:
            attn_fixture(*f)
        return
    layer_fixture("cfg1_layer_f32", CFG1, seed=0, T=64, int8=False, zero_state=True, gnorm_std=0.0)
    layer_fixture("tiny_layer_int8", TINY, seed=1, T=65, int8=True, zero_state=False, gnorm_std=0.1)
    core_fixture("core_rep3_d16", GdnDims(2, 6, 16, 16, 4, 0), seed=2, T=33, gnorm_std=0.1)
    core_fixture("core_kd32_vd16", GdnDims(2, 4, 32, 16, 4, 0), seed=4, T=17, gnorm_std=0.1)
    core_fixture("core_d128", GdnDims(1, 2, 128, 128, 4, 0), seed=3, T=5, gnorm_std=0.1)
    core_fixture("core_d32_decay", GdnDims(2, 4, 32, 32, 4, 0), seed=5, T=70, gnorm_std=0.1,
                 a_mean=2.0)
    quant_fixture("quant_rows")
    for f in ATTN_FIXTURES:
        attn_fixture(*f)
    copy_tiny_model()


if __name__ == "__main__":
    main()
