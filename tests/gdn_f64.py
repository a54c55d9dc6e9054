"""Float64 matrix-form GDN recurrence (test checker).

Written from the mathematics of the gated delta rule, not from the loop nest
of the reference: the conv is a sliding window product, the recurrence uses
whole-matrix numpy operations.  It is the independent check that the C
restatement (oracle/) and the chunked algebra agree with the textbook form:

    conv:  u_t = sum_j w[:, j] * window_t[:, j];  c_t = silu(u_t)
    norm:  q = c_q / |c_q| / sqrt(kd),  k = c_k / |c_k|   (eps 1e-6 inside the root)
    gates: g = -exp(A_log) softplus(a + dt_bias),  beta = sigmoid(b)
    rule:  S <- e^g S;  S <- S + beta k (v - S^T k)^T;  o = S^T q
    norm:  y = o / sqrt(mean(o^2) + eps) * gnorm * silu(z)
"""
from __future__ import annotations

import numpy as np


def _silu(x):
    return x / (1.0 + np.exp(-x))


def _softplus(x):
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def prepare(d, w, inp, conv0):
    """Conv + SiLU + norms + gates for T tokens.  Returns per-token float64
    q [T][kh][kd] (normalised, scaled), k [T][kh][kd], v [T][vh][vd],
    g [T][vh], beta [T][vh], z [T][vh][vd], and the final conv window."""
    qkv = np.asarray(inp["qkv"], np.float64)
    T = qkv.shape[0]
    K = d.K
    hist = np.concatenate([np.asarray(conv0, np.float64), qkv.T], axis=1)  # [conv_dim][K-1+T]
    wc = np.asarray(w["conv_w"], np.float64)
    u = np.stack([(hist[:, t:t + K] * wc).sum(axis=1) for t in range(T)])  # [T][conv_dim]
    c = _silu(u)
    kdim = d.kh * d.kd
    q = c[:, :kdim].reshape(T, d.kh, d.kd)
    k = c[:, kdim:2 * kdim].reshape(T, d.kh, d.kd)
    v = c[:, 2 * kdim:].reshape(T, d.vh, d.vd)
    q = q / np.sqrt((q * q).sum(-1, keepdims=True) + 1e-6) / np.sqrt(d.kd)
    k = k / np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    a = np.asarray(inp["a"], np.float64)
    b = np.asarray(inp["b"], np.float64)
    g = -np.exp(np.asarray(w["A_log"], np.float64)) * _softplus(a + np.asarray(w["dt_bias"], np.float64))
    beta = 1.0 / (1.0 + np.exp(-b))
    z = np.asarray(inp["z"], np.float64).reshape(T, d.vh, d.vd)
    conv_final = hist[:, -(K - 1):]
    return q, k, v, g, beta, z, conv_final


def recurrence(d, q, k, v, g, beta, S0):
    """Un-normalised outputs o [T][vh][vd] and final S [vh][kd][vd]."""
    T = q.shape[0]
    rep = d.vh // d.kh
    S = np.array(S0, np.float64, copy=True)
    o = np.zeros((T, d.vh, d.vd))
    for t in range(T):
        for h in range(d.vh):
            kk, qq = k[t, h // rep], q[t, h // rep]
            S[h] *= np.exp(g[t, h])
            S[h] += beta[t, h] * np.outer(kk, v[t, h] - S[h].T @ kk)
            o[t, h] = S[h].T @ qq
    return o, S


def gated_norm(d, o, z, gnorm):
    r = 1.0 / np.sqrt((o * o).mean(-1, keepdims=True) + d.eps)
    return o * r * np.asarray(gnorm, np.float64) * _silu(z)


def core(d, w, inp, conv0, S0):
    """Full core in float64: returns (core [T][vh*vd], o_raw, S_final, conv_final)."""
    q, k, v, g, beta, z, conv_final = prepare(d, w, inp, conv0)
    o, S = recurrence(d, q, k, v, g, beta, S0)
    y = gated_norm(d, o, z, w["gnorm"])
    return y.reshape(y.shape[0], -1), o, S, conv_final
