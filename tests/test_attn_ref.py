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
