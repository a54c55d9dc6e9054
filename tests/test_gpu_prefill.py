"""GPU parity of the chunked prefill through the C-ABI.

The reference engine prefills token by token (overhang engines/qwen.c:588,
637); the chunked form must agree with that recurrence (the CPU oracle, and
the reference's own golden vectors) on outputs and final state, at every
length around the 64-token chunk boundary, across split points, mixed with
decode steps, at the Qwen3.6-35B-A3B shape up to T=4096, and under strong
decay.  Tolerance: tests/tol.py."""
import numpy as np
import pytest

import oracle
from overhang_amd import gdn, synth
from overhang_amd.dims import GdnDims, Q35B, CFG1, TINY
from tests import fixtures
from tests.tol import assert_close

pytestmark = pytest.mark.gpu

_next_li = [500]


def new_li():
    _next_li[0] += 1
    return _next_li[0]


def _layer(d, seed, gnorm_std=0.1, max_seqs=1):
    w = synth.layer_weights(d, seed, gnorm_std=gnorm_std, projections=False)
    conv0, S0 = synth.states(d, seed)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=max_seqs)
    L.set_state(0, conv0, S0)
    return L, w, conv0, S0


@pytest.mark.parametrize("D", [16, 32, 64, 128])
@pytest.mark.parametrize("T", [1, 3, 63, 64, 65, 130])
def test_prefill_matches_recurrent_oracle(D, T):
    d = GdnDims(2, 4, D, D, 4, 0)
    seed = 1000 + D + T
    L, w, conv0, S0 = _layer(d, seed)
    inp = synth.core_inputs(d, T, seed)
    core = L.prefill_core(0, inp["qkv"], inp["z"], inp["a"], inp["b"])
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    conv, S = L.get_state(0)
    assert_close(core, ref, what=f"D={D} T={T} core")
    assert_close(S, Sref, what=f"D={D} T={T} S")
    assert np.array_equal(conv, cref), "conv history is a copy of the inputs"
    L.free()


@pytest.mark.parametrize("kh,vh,D,K", [(2, 2, 64, 4), (1, 3, 32, 4), (1, 4, 64, 4), (2, 8, 128, 4), (1, 6, 16, 4),
                                        (2, 4, 32, 3), (2, 4, 32, 2), (1, 2, 128, 3)])
@pytest.mark.parametrize("T", [65, 200])
def test_prefill_head_groupings_and_conv_widths(kh, vh, D, K, T):
    """The WY kernel takes a key head's value heads two at a time when their
    number is even, one at a time otherwise (rep 1, 3), in several groups
    when there are more (rep 4, 6); conv widths 2-4 are separate kernels."""
    d = GdnDims(kh, vh, D, D, K, 0)
    seed = 3000 + 7 * kh + vh + D + K + T
    L, w, conv0, S0 = _layer(d, seed)
    inp = synth.core_inputs(d, T, seed)
    core = L.prefill_core(0, inp["qkv"], inp["z"], inp["a"], inp["b"])
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    conv, S = L.get_state(0)
    what = f"kh={kh} vh={vh} D={D} K={K} T={T}"
    assert_close(core, ref, what=what + " core")
    assert_close(S, Sref, what=what + " S")
    assert np.array_equal(conv, cref), "conv history is a copy of the inputs"
    L.free()


@pytest.mark.parametrize("name", ["core_rep3_d16", "core_d128", "core_d32_decay"])
def test_prefill_matches_reference_golden(name):
    d, w, inp, (conv, S), exp = fixtures.load(name)
    L = gdn.GdnLayer(new_li(), d, w)
    L.set_state(0, conv, S)
    core = L.prefill_core(0, inp["qkv"], inp["z"], inp["a"], inp["b"])
    conv2, S2 = L.get_state(0)
    assert_close(core, exp["core"], what=f"{name} core")
    assert_close(S2, exp["S"], what=f"{name} S")
    assert np.array_equal(conv2, exp["conv"])
    L.free()


@pytest.mark.parametrize("name", fixtures.LAYER_FIXTURES)
def test_full_layer_prefill_matches_reference_golden(name):
    d, w, inp, (conv, S), exp = fixtures.load(name)
    L = gdn.GdnLayer(new_li(), d, w, int8=exp["int8"])
    L.set_state(0, conv, S)
    out = L.prefill(0, inp["x"])
    conv2, S2 = L.get_state(0)
    assert_close(out, exp["out"], what=f"{name} out")
    assert_close(S2, exp["S"], what=f"{name} S")
    assert_close(conv2, exp["conv"], atol=1e-5, rtol=1e-5)
    L.free()


def test_unsupported_prefill_shape_is_rejected():
    d, w, inp, (conv, S), exp = fixtures.load("core_kd32_vd16")
    L = gdn.GdnLayer(new_li(), d, w)
    with pytest.raises(gdn.OmhError) as e:
        L.prefill_core(0, inp["qkv"], inp["z"], inp["a"], inp["b"])
    assert e.value.code == gdn.OMH_ERR_SHAPE
    L.free()


@pytest.mark.parametrize("split", [[1, 199], [64, 136], [100, 37, 63], [5, 5, 5, 185]])
def test_split_invariance_and_decode_interleave(split):
    """prefill(T1); prefill(T2); ... == one recurrent pass over T1+T2+...,
    with a decode step between the pieces."""
    d = GdnDims(2, 4, 32, 32, 4, 0)
    seed = 2000 + sum(split) + len(split)
    L, w, conv0, S0 = _layer(d, seed)
    T = sum(split) + len(split) - 1
    inp = synth.core_inputs(d, T, seed)
    got, t = [], 0
    for i, n in enumerate(split):
        sl = slice(t, t + n)
        got.append(L.prefill_core(0, inp["qkv"][sl], inp["z"][sl], inp["a"][sl], inp["b"][sl]))
        t += n
        if i < len(split) - 1:
            sl = slice(t, t + 1)
            got.append(L.decode_core(inp["qkv"][sl], inp["z"][sl], inp["a"][sl], inp["b"][sl]))
            t += 1
    got = np.concatenate(got)
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    conv, S = L.get_state(0)
    assert_close(got, ref, what=f"split {split}")
    assert_close(S, Sref, what=f"split {split} S")
    assert np.array_equal(conv, cref)
    L.free()


def test_prefill_leaves_other_sequences_alone():
    d = CFG1
    w = synth.layer_weights(d, 3000, projections=False)
    conv0, S0 = synth.states(d, 3000, B=3)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=3)
    for s in range(3):
        L.set_state(s, conv0[s], S0[s])
    inp = synth.core_inputs(d, 70, 3001)
    core = L.prefill_core(1, inp["qkv"], inp["z"], inp["a"], inp["b"])
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0[1], S0[1])
    assert_close(core, ref)
    for s in (0, 2):
        c, S = L.get_state(s)
        assert np.array_equal(c, conv0[s]) and np.array_equal(S, S0[s])
    # a batched decode of all three afterwards continues each sequence correctly
    nxt = synth.core_inputs(d, 1, 3002, B=3)
    out = L.decode_core(nxt["qkv"][:, 0], nxt["z"][:, 0], nxt["a"][:, 0], nxt["b"][:, 0])
    starts = {0: (conv0[0], S0[0]), 1: (cref, Sref), 2: (conv0[2], S0[2])}
    for s in range(3):
        r, _, _ = oracle.core_seq(d, w, nxt["qkv"][s], nxt["z"][s], nxt["a"][s], nxt["b"][s], *starts[s])
        assert_close(out[s:s + 1], r, what=f"seq {s} decode after prefill")
    L.free()


@pytest.mark.parametrize("T", [300, 4096])
def test_prefill_35b_shape(T):
    """Qwen3.6-35B-A3B GDN shape (16 key / 32 value heads, d=128); T=4096 is
    the prefill benchmark's length."""
    d = Q35B
    seed = 4000 + T
    L, w, conv0, S0 = _layer(d, seed)
    inp = synth.core_inputs(d, T, seed)
    core = L.prefill_core(0, inp["qkv"], inp["z"], inp["a"], inp["b"])
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    conv, S = L.get_state(0)
    assert_close(core, ref, what=f"35B T={T} core")
    assert_close(S, Sref, what=f"35B T={T} S")
    assert np.array_equal(conv, cref)
    L.free()


def test_prefill_strong_decay():
    """Gate logits a ~ N(2, 1) with A_log = ln 16: per-chunk cumulative decay
    far below exp(-100); only decay differences are exponentiated."""
    d = GdnDims(2, 4, 64, 64, 4, 0)
    w = synth.layer_weights(d, 5000, gnorm_std=0.1, projections=False)
    w["A_log"][:] = np.log(16.0)
    conv0, S0 = synth.states(d, 5000)
    L = gdn.GdnLayer(new_li(), d, w)
    L.set_state(0, conv0, S0)
    T = 400
    inp = synth.core_inputs(d, T, 5000, a_mean=2.0)
    core = L.prefill_core(0, inp["qkv"], inp["z"], inp["a"], inp["b"])
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    assert np.isfinite(core).all()
    assert_close(core, ref, what="strong decay core")
    assert_close(L.get_state(0)[1], Sref, what="strong decay S")
    L.free()


def test_long_warm_append_matches_recurrent_oracle():
    """Config 4 at reduced width: 8192 tokens of warm-up, then a 32768-token
    prefill continuing from that state, gate logits a ~ N(-2, 1); one key
    head / two value heads of the 35B head dims (d=128), so the recurrent
    oracle finishes in seconds."""
    d = GdnDims(1, 2, 128, 128, 4, 0)
    seed = 6000
    L, w, conv0, S0 = _layer(d, seed)
    Tw, T = 8192, 32768
    inp = synth.core_inputs(d, Tw + T, seed, a_mean=-2.0)
    part = lambda lo, hi: [inp[k][lo:hi] for k in ("qkv", "z", "a", "b")]
    L.prefill_core(0, *part(0, Tw))
    got = L.prefill_core(0, *part(Tw, Tw + T))
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    conv, S = L.get_state(0)
    assert_close(got, ref[Tw:], what="warm-append core")
    assert_close(S, Sref, what="warm-append S")
    assert np.array_equal(conv, cref)
    L.free()


def _key_head_slice(d, w, inp, conv0, S0, j):
    """The layer restricted to key head j and its value heads: their conv
    channels (q and k of key head j, v of its value heads), gates, z
    columns and states.  The core couples nothing across key-head groups
    (qwen.c:331-357: each value head reads only its key head's q, k), so the
    oracle on this one-key-head layer gives the full layer's values for
    those heads."""
    kd, vd, rep = d.kd, d.vd, d.vh // d.kh
    key_dim = d.kh * kd
    hs = np.arange(j * rep, (j + 1) * rep)
    ch = np.r_[j * kd:(j + 1) * kd, key_dim + j * kd:key_dim + (j + 1) * kd,
               2 * key_dim + j * rep * vd:2 * key_dim + (j + 1) * rep * vd]
    zc = np.arange(j * rep * vd, (j + 1) * rep * vd)
    ds = GdnDims(1, rep, kd, vd, d.K, 0)
    ws = {"conv_w": np.ascontiguousarray(w["conv_w"][ch]), "A_log": w["A_log"][hs], "dt_bias": w["dt_bias"][hs],
          "gnorm": w["gnorm"]}
    ins = [np.ascontiguousarray(inp["qkv"][:, ch]), np.ascontiguousarray(inp["z"][:, zc]),
           np.ascontiguousarray(inp["a"][:, hs]), np.ascontiguousarray(inp["b"][:, hs])]
    return ds, ws, ins, np.ascontiguousarray(conv0[ch]), np.ascontiguousarray(S0[hs]), hs, ch, zc


def test_long_warm_append_35b_full_width_vs_oracle():
    """Config 4 at the full 35B-A3B width (16 key / 32 value heads): an
    8192-token prefill, then 32768 tokens continuing from its state, gate
    logits a ~ N(-2, 1), every input seeded over all 40960 tokens (no
    repeated block).  The oracle recurrence runs over three key-head groups
    of the same layer (key heads 0, 9, 15 with their value heads, sliced out
    as one-key-head layers), token by token over all 40960 tokens; their
    outputs of the 32768-token call, final states and conv histories must
    match."""
    d = Q35B
    seed = 6200
    L, w, conv0, S0 = _layer(d, seed)
    Tw, T = 8192, 32768
    # (numpy's generator: 335 M normals in seconds, where the repository's
    # splitmix64 generator takes a minute)
    rng = np.random.default_rng(seed)
    N = Tw + T
    inp = {"qkv": rng.standard_normal((N, d.conv_dim), dtype=np.float32),
           "z": rng.standard_normal((N, d.val_dim), dtype=np.float32),
           "a": rng.standard_normal((N, d.vh), dtype=np.float32) - np.float32(2.0),
           "b": rng.standard_normal((N, d.vh), dtype=np.float32)}
    part = lambda lo, hi: [np.ascontiguousarray(inp[k][lo:hi]) for k in ("qkv", "z", "a", "b")]
    L.prefill_core(0, *part(0, Tw))
    got = L.prefill_core(0, *part(Tw, Tw + T))
    conv, S = L.get_state(0)
    L.free()
    for j in (0, 9, 15):
        ds, ws, ins, c0, s0, hs, ch, zc = _key_head_slice(d, w, inp, conv0, S0, j)
        ref, cref, Sref = oracle.core_seq(ds, ws, *ins, c0, s0)
        assert_close(got[:, zc], ref[Tw:], what=f"35B warm-append key head {j} core")
        assert_close(S[hs], Sref, what=f"35B warm-append key head {j} S")
        assert np.array_equal(conv[ch], cref), f"key head {j} conv history"


@pytest.mark.parametrize("split", [8192, 8200])
def test_long_warm_append_35b_split_invariance(split):
    """Config 4 at the 35B shape: prefill(split) then prefill(40960 - split)
    equals one 40960-token prefill from the same state (bit-identical when the
    split falls on a chunk boundary).  Inputs are a 4096-token seeded block
    repeated, a ~ N(-2, 1)."""
    d = Q35B
    seed = 6100
    w = synth.layer_weights(d, seed, gnorm_std=0.1, projections=False)
    conv0, S0 = synth.states(d, seed)
    blk = synth.core_inputs(d, 4096, seed, a_mean=-2.0)
    N = 40960
    inp = {k: np.ascontiguousarray(np.tile(v, (N // 4096, 1))) for k, v in blk.items()}
    part = lambda lo, hi: [inp[k][lo:hi] for k in ("qkv", "z", "a", "b")]
    A = gdn.GdnLayer(new_li(), d, w)
    B = gdn.GdnLayer(new_li(), d, w)
    for L in (A, B):
        L.set_state(0, conv0, S0)
    one = A.prefill_core(0, *part(0, N))
    two = np.concatenate([B.prefill_core(0, *part(0, split)), B.prefill_core(0, *part(split, N))])
    (ca, Sa), (cb, Sb) = A.get_state(0), B.get_state(0)
    assert np.array_equal(ca, cb)
    if split % 64 == 0:
        assert np.array_equal(one, two) and np.array_equal(Sa, Sb), "chunk-aligned split must be bit-identical"
    else:
        assert_close(two, one, what=f"split {split} core")
        assert_close(Sb, Sa, what=f"split {split} S")
    A.free()
    B.free()
