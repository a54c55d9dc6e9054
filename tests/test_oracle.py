"""Pins the CPU oracle (oracle/gdn_oracle.c) before anything is checked against it.

1. Golden vectors written by the reference engine's own deltanet_step
   (tests/golden/make_golden.py, overhang engines/qwen.c:301-364): bit-exact.
2. The compiled reference itself (oracle/_ref), where it was built: bit-exact
   on fresh random cases.
3. Mathematics: closed forms that a dropped term, a wrong sign, a swapped
   index or a transposed state would break, an independent float64
   matrix-form recurrence, and the chunked (WY/UT) algebra against it.
"""
import numpy as np
import pytest

import oracle
from overhang_amd import synth
from overhang_amd.dims import GdnDims, CFG1, TINY
from tests import fixtures, gdn_f64


@pytest.mark.parametrize("name", fixtures.LAYER_FIXTURES)
def test_layer_matches_reference_golden(name):
    d, w, inp, (conv, S), exp = fixtures.load(name)
    out, conv2, S2 = oracle.layer_seq(d, w, inp["x"], conv, S, int8=exp["int8"])
    assert np.array_equal(out, exp["out"])
    assert np.array_equal(conv2, exp["conv"])
    assert np.array_equal(S2, exp["S"])


@pytest.mark.parametrize("name", fixtures.CORE_FIXTURES)
def test_core_matches_reference_golden(name):
    d, w, inp, (conv, S), exp = fixtures.load(name)
    core, conv2, S2 = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv, S)
    assert np.array_equal(core, exp["core"])
    assert np.array_equal(conv2, exp["conv"])
    assert np.array_equal(S2, exp["S"])


def test_quantizer_and_int8_matvec_golden():
    f = np.load(fixtures.GOLDEN + "/quant_rows.npz", allow_pickle=False)
    q, s = oracle.quantize_rows(f["W"])
    assert np.array_equal(q, f["q"]) and np.array_equal(s, f["s"])
    assert np.array_equal(oracle.matmul_q(f["x"], q, s), f["y"])
    assert np.array_equal(oracle.matvec(f["x"], f["W"]), f["yf"])
    # closed forms: zero row -> floor scale and zeros; absmax maps to +-127
    assert s[6] == np.float32(1e-8) and not q[6].any()
    assert np.abs(q[:6]).max(axis=1).tolist() == [127] * 6
    # int8 dequant against float64 brute force
    ref = (f["x"].astype(np.float64) @ q.astype(np.float64).T) * s
    np.testing.assert_allclose(f["y"], ref, rtol=1e-5, atol=1e-9)


@pytest.mark.skipif(oracle.ref_lib() is None, reason="reference not compiled (oracle/_ref)")
@pytest.mark.parametrize("int8", [False, True])
def test_random_cases_match_compiled_reference(int8):
    for seed, d in [(11, GdnDims(2, 6, 16, 16, 4, 48)), (12, GdnDims(1, 1, 64, 32, 3, 96))]:
        w = synth.layer_weights(d, seed, gnorm_std=0.2, proj_std=0.1)
        x = synth.normal(seed, synth.S_X, (9, d.hidden))
        conv, S = synth.states(d, seed)
        a = oracle.layer_seq(d, w, x, conv, S, int8=int8)
        b = oracle.ref_layer_seq(d, w, x, conv, S, int8=int8)
        for u, v in zip(a, b):
            assert np.array_equal(u, v)


def _zero_states(d):
    return (np.zeros((d.conv_dim, d.K - 1), np.float32), np.zeros((d.vh, d.kd, d.vd), np.float32))


def test_closed_form_first_token_from_zero_state():
    """S0 = 0, conv0 = 0: only the last conv tap sees the input, kv = 0, so
    S1 = beta k v^T (per v-head, with its k-head h // rep) and
    o = beta (q.k) v, then the gated norm."""
    d = GdnDims(2, 4, 16, 8, 4, 0)
    w = synth.layer_weights(d, 21, gnorm_std=0.3, projections=False)
    inp = synth.core_inputs(d, 1, 21)
    conv0, S0 = _zero_states(d)
    core, conv1, S1 = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    x = inp["qkv"][0].astype(np.float64)
    c = x * w["conv_w"][:, -1]
    c = c / (1 + np.exp(-c))
    kdim = d.kh * d.kd
    rep = d.vh // d.kh
    beta = 1 / (1 + np.exp(-inp["b"][0].astype(np.float64)))
    for h in range(d.vh):
        hk = h // rep
        q = c[hk * d.kd:(hk + 1) * d.kd]
        k = c[kdim + hk * d.kd:kdim + (hk + 1) * d.kd]
        v = c[2 * kdim + h * d.vd:2 * kdim + (h + 1) * d.vd]
        qh = q / np.sqrt((q * q).sum() + 1e-6) / np.sqrt(d.kd)
        kh_ = k / np.sqrt((k * k).sum() + 1e-6)
        np.testing.assert_allclose(S1[h], beta[h] * np.outer(kh_, v), rtol=2e-5, atol=1e-7)
        o = beta[h] * (qh @ kh_) * v
        zz = inp["z"][0, h * d.vd:(h + 1) * d.vd].astype(np.float64)
        y = o / np.sqrt((o * o).mean() + d.eps) * w["gnorm"] * zz / (1 + np.exp(-zz))
        np.testing.assert_allclose(core[0, h * d.vd:(h + 1) * d.vd], y, rtol=2e-4, atol=2e-6)
    # conv window now holds [0, 0, x]
    assert np.array_equal(conv1[:, -1], inp["qkv"][0]) and not conv1[:, :-1].any()


def test_closed_form_beta_zero_is_pure_decay():
    """beta = 0 (b = -100): S_T = exp(sum_t g_t) S_0 with g from A_log, a, dt_bias."""
    d = GdnDims(2, 4, 16, 16, 4, 0)
    w = synth.layer_weights(d, 22, projections=False)
    T = 7
    inp = synth.core_inputs(d, T, 22)
    inp["b"][:] = -100.0
    conv0, S0 = synth.states(d, 22)
    _, _, S = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    x = inp["a"].astype(np.float64) + w["dt_bias"]
    g = -np.exp(w["A_log"].astype(np.float64)) * np.log1p(np.exp(x))
    decay = np.exp(g.sum(0))
    np.testing.assert_allclose(S, decay[:, None, None] * S0, rtol=3e-6, atol=1e-30)


def test_closed_form_retrieval_beta_one_no_decay():
    """beta = 1, gamma = 1: after the update S'^T k = v exactly (|k| = 1)."""
    d = GdnDims(1, 1, 32, 16, 4, 0)
    w = synth.layer_weights(d, 23, projections=False)
    inp = synth.core_inputs(d, 1, 23)
    inp["b"][:] = 100.0
    inp["a"][:] = -100.0
    conv0, S0 = synth.states(d, 23, s_std=0.3)
    _, _, S1 = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    q, k, v, g, beta, z, _ = gdn_f64.prepare(d, w, inp, conv0)
    assert beta[0, 0] == 1.0 and g[0, 0] > -1e-30
    np.testing.assert_allclose(S1[0].astype(np.float64).T @ k[0, 0], v[0, 0], rtol=1e-5, atol=1e-5)


def test_gate_zero_gives_zero_output():
    d = CFG1
    w = synth.layer_weights(d, 24, projections=False)
    inp = synth.core_inputs(d, 3, 24)
    inp["z"][:] = 0.0
    conv0, S0 = synth.states(d, 24)
    core, _, _ = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    assert not core.any()


@pytest.mark.parametrize("d", [TINY, CFG1, GdnDims(2, 6, 16, 8, 4, 0)])
def test_oracle_matches_float64_matrix_form(d):
    w = synth.layer_weights(d, 25, gnorm_std=0.2, projections=False)
    T = 40
    inp = synth.core_inputs(d, T, 25)
    conv0, S0 = synth.states(d, 25)
    core, conv, S = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    y, _, S64, conv64 = gdn_f64.core(d, w, inp, conv0, S0)
    np.testing.assert_allclose(core, y, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(S, S64, rtol=1e-4, atol=1e-6)
    assert np.array_equal(conv, conv64.astype(np.float32))


@pytest.mark.parametrize("T,C", [(1, 64), (63, 64), (65, 64), (130, 64), (130, 32), (97, 16)])
def test_chunked_algebra_matches_recurrence(T, C):
    d = GdnDims(2, 4, 16, 16, 4, 0)
    w = synth.layer_weights(d, 26, projections=False)
    inp = synth.core_inputs(d, T, 26)
    conv0, S0 = synth.states(d, 26)
    q, k, v, g, beta, z, _ = gdn_f64.prepare(d, w, inp, conv0)
    o64, S64 = gdn_f64.recurrence(d, q, k, v, g, beta, S0)
    f = np.float32
    o, S = oracle.chunked(d, q.astype(f), k.astype(f), v.astype(f), g.astype(f),
                          beta.astype(f), S0, C)
    np.testing.assert_allclose(o, o64, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(S, S64, rtol=1e-4, atol=1e-6)


def test_chunked_strong_decay_is_finite():
    """a ~ N(2, 1) gives cumulative log-decay of order -100 per chunk: only
    differences of cumulative g are exponentiated, so nothing overflows."""
    d = GdnDims(1, 2, 16, 16, 4, 0)
    w = synth.layer_weights(d, 27, projections=False)
    w["A_log"][:] = np.log(16.0)
    T = 128
    inp = synth.core_inputs(d, T, 27, a_mean=2.0)
    conv0, S0 = synth.states(d, 27)
    q, k, v, g, beta, z, _ = gdn_f64.prepare(d, w, inp, conv0)
    assert g.sum(0).min() < -1000
    o64, S64 = gdn_f64.recurrence(d, q, k, v, g, beta, S0)
    f = np.float32
    o, S = oracle.chunked(d, q.astype(f), k.astype(f), v.astype(f), g.astype(f),
                          beta.astype(f), S0, 64)
    assert np.isfinite(o).all() and np.isfinite(S).all()
    np.testing.assert_allclose(o, o64, rtol=1e-4, atol=1e-5)
