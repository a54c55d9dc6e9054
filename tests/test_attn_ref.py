"""Closed-form checks of tests/qwen_tiny.gated_attention, the float32
restatement of the engine's attn_step (engines/qwen.c:366-425) that the GPU
attention layer is compared with.  Beside the token-level pin (the host
model with it reproduces the reference's greedy and teacher-forced golden
tokens, test_e2e_tiny.py), two cases reduce it to arithmetic that does not
go through its own formula:
  - the first token (pos 0) sees one key, so its softmax weight is 1 and the
    output is v * sigmoid(gate) through o_proj, for every query head of a
    group (the h // grp mapping, qwen.c:408-409);
  - with q_norm = -1 the (1 + w) norm weight is 0, every score is 0, and
    token t averages v over positions 0..t: the causal mask and the weights'
    normalisation (qwen.c:410-419)."""
import numpy as np

from tests import qwen_tiny as q


def _w(rng, D, H, KV, hd):
    return {"q_proj": rng.normal(0, 0.1, (2 * H * hd, D)).astype(np.float32),
            "k_proj": rng.normal(0, 0.1, (KV * hd, D)).astype(np.float32),
            "v_proj": rng.normal(0, 0.1, (KV * hd, D)).astype(np.float32),
            "o_proj": rng.normal(0, 0.1, (D, H * hd)).astype(np.float32),
            "q_norm": rng.normal(0, 0.1, hd).astype(np.float32),
            "k_norm": rng.normal(0, 0.1, hd).astype(np.float32)}


def _gated_v(x, W, H, KV, hd):
    """v of each token's kv head times sigmoid(gate), per query head [T][H*hd]."""
    T = x.shape[0]
    g = (x.astype(np.float64) @ W["q_proj"].T.astype(np.float64)).reshape(T, H, 2 * hd)[:, :, hd:]
    v = (x.astype(np.float64) @ W["v_proj"].T.astype(np.float64)).reshape(T, KV, hd)
    return v, 1.0 / (1.0 + np.exp(-g))


def test_first_token_attends_to_itself_only():
    D, H, KV, hd, rot = 32, 4, 2, 16, 8
    rng = np.random.default_rng(0)
    W = _w(rng, D, H, KV, hd)
    x = rng.normal(0, 1, (1, D)).astype(np.float32)
    got = q.gated_attention(x, W, [], [], 0, H, KV, hd, rot, 1e7, 1e-6)
    v, sg = _gated_v(x, W, H, KV, hd)
    ctx = np.stack([v[0, h // (H // KV)] * sg[0, h] for h in range(H)]).reshape(1, H * hd)
    exp = ctx @ W["o_proj"].T.astype(np.float64)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6)


def test_zero_queries_average_values_causally():
    D, H, KV, hd, rot = 32, 6, 3, 16, 16
    rng = np.random.default_rng(1)
    W = _w(rng, D, H, KV, hd)
    W["q_norm"] = np.full(hd, -1.0, np.float32)         # (1 + w) = 0: q = 0
    x = rng.normal(0, 1, (5, D)).astype(np.float32)
    Kl, Vl = [], []
    got = np.concatenate([q.gated_attention(x[:2], W, Kl, Vl, 0, H, KV, hd, rot, 1e7, 1e-6),
                          q.gated_attention(x[2:], W, Kl, Vl, 2, H, KV, hd, rot, 1e7, 1e-6)])
    v, sg = _gated_v(x, W, H, KV, hd)
    grp = H // KV
    ctx = np.stack([np.stack([v[:t + 1, h // grp].mean(axis=0) * sg[t, h] for h in range(H)]).reshape(H * hd)
                    for t in range(5)])
    exp = ctx @ W["o_proj"].T.astype(np.float64)
    np.testing.assert_allclose(got, exp, rtol=1e-5, atol=1e-6)


# ---- against the reference's own attn_step ----

import hashlib  # noqa: E402
import os  # noqa: E402

import pytest  # noqa: E402

import oracle  # noqa: E402
from overhang_amd import gdn, synth  # noqa: E402

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ATTN_FIXTURES = ["attn_tiny_f32", "attn_tiny_int8", "attn_35b_f32", "attn_35b_int8"]


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def load_attn(name):
    """(shape, weights as the checker takes them, x, Kpre, Vpre, expected):
    inputs regenerated from overhang_amd.synth and hash-checked against the
    fixture, which tests/golden/make_golden.py wrote from the reference's
    attn_step (qwen.c:367-425)."""
    f = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    D, H, KV, hd, rot, pos0, T = (int(v) for v in f["dims"])
    seed, int8 = int(f["seed"]), bool(int(f["int8"]))
    w = synth.attn_weights(D, H, KV, hd, seed)
    x, Kpre, Vpre = synth.attn_inputs(D, KV, hd, pos0, T, seed)
    for k, v in list(w.items()) + [("x", x), ("Kpre", Kpre), ("Vpre", Vpre)]:
        assert _sha(v) == str(f["sha_" + k]), f"{name}: regenerated {k} differs from the fixture's"
    shape = dict(D=D, H=H, KV=KV, hd=hd, rot=rot, pos0=pos0, T=T, theta=float(f["theta"]),
                 eps=float(f["eps"]), int8=int8)
    exp = {"out": f["out"], "K": f["K"], "V": f["V"]}
    return shape, w, x, Kpre, Vpre, exp


def checker_weights(w, int8):
    """The checker's weight dict; for int8, the values the engine's matmul_q
    multiplies by: q * s per row (qwen.c:116-121)."""
    if int8:
        w = dict(w)
        for nm in ("q", "k", "v", "o"):
            Q, S = gdn.quantize_rows(w["W_" + nm])
            w["W_" + nm] = (Q.astype(np.float32) * S[:, None]).astype(np.float32)
    return {"q_proj": w["W_q"], "k_proj": w["W_k"], "v_proj": w["W_v"], "o_proj": w["W_o"],
            "q_norm": w["q_norm"], "k_norm": w["k_norm"]}


def _close(got, exp, what):
    # float32 sums in another order (BLAS vs the engine's loops): ~1e-6 relative
    scale = float(np.abs(exp).max())
    err = float(np.abs(got - exp).max())
    assert err <= 2e-5 * max(scale, 1e-3) + 1e-7, f"{what}: max err {err:.3g} at scale {scale:.3g}"


@pytest.mark.parametrize("name", ATTN_FIXTURES)
def test_checker_matches_reference_attn_golden(name):
    """The attention checker against the reference's attn_step at positions
    in the thousands (partial RoPE at large angles, the q/k (1 + w) norms,
    GQA, the causal softmax over a prefilled cache), fp32 and int8."""
    s, w, x, Kpre, Vpre, exp = load_attn(name)
    Kl, Vl = [Kpre], [Vpre]
    got = q.gated_attention(x, checker_weights(w, s["int8"]), Kl, Vl, s["pos0"], s["H"], s["KV"], s["hd"],
                            s["rot"], s["theta"], s["eps"])
    _close(got, exp["out"], f"{name} out")
    _close(Kl[-1], exp["K"], f"{name} K rows")
    _close(Vl[-1], exp["V"], f"{name} V rows")


def test_checker_matches_live_reference_attn():
    """Fresh random cases through the compiled reference (where it is built):
    a 5-token prompt from position 0, then one token at position 3001."""
    if oracle.ref_lib() is None:
        pytest.skip("oracle/_ref not built (reference sources absent at build time)")
    D, H, KV, hd, rot = 96, 6, 2, 64, 16
    for int8 in (False, True):
        w = synth.attn_weights(D, H, KV, hd, 21 + int8)
        x, Kpre, Vpre = synth.attn_inputs(D, KV, hd, 3001, 5, 21 + int8)
        cw = checker_weights(w, int8)
        out, Kn, Vn = oracle.ref_attn_run(w, H, KV, hd, rot, 1e7, 1e-6, 0, None, None, x, int8=int8)
        got = q.gated_attention(x, cw, [], [], 0, H, KV, hd, rot, 1e7, 1e-6)
        _close(got, out, f"int8={int8} prompt")
        out, Kn, Vn = oracle.ref_attn_run(w, H, KV, hd, rot, 1e7, 1e-6, 3001, Kpre, Vpre, x[:1], int8=int8)
        got = q.gated_attention(x[:1], cw, [Kpre], [Vpre], 3001, H, KV, hd, rot, 1e7, 1e-6)
        _close(got, out, f"int8={int8} pos 3001")


def test_attn_fixture_catches_a_dropped_rope():
    """The fixtures see RoPE: a checker variant without the rotation (planted
    here on the CPU) misses the 35B fixture by far more than the tolerance."""
    s, w, x, Kpre, Vpre, exp = load_attn("attn_35b_f32")
    got = q.gated_attention(x, checker_weights(w, False), [Kpre], [Vpre], s["pos0"], s["H"], s["KV"],
                            s["hd"], 0, s["theta"], s["eps"])
    assert float(np.abs(got - exp["out"]).max()) > 1e-3 * float(np.abs(exp["out"]).max())
