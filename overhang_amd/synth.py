"""Deterministic synthetic inputs for the GDN path.

Counter-based splitmix64 turned into uniforms (53-bit) and, through
Box-Muller, into normals.  Every tensor draws from its own stream
``(seed, stream)``, so adding or resizing one tensor never shifts another.
Values are computed in float64 and rounded once to float32, so the same
arrays come out on any machine with IEEE float64.

The layer-weight distributions follow the benchmark definitions for the
Qwen3.5/3.6 GDN layer: projections N(0, 0.02), conv1d N(0, 0.1),
A_log U[0, ln 16], dt_bias N(0, 0.1), gated-norm weight 1 (the transformers
initialisation, modeling_qwen3_5_moe.py:172) unless ``gnorm_std`` is given.
"""
from __future__ import annotations

import math

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_CHUNK = 1 << 22


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def _base(seed: int, stream: int) -> np.uint64:
    with np.errstate(over="ignore"):
        s = _mix(np.array([(seed * 0x100000001B3 + stream * 0x9E37) & 0xFFFFFFFFFFFFFFFF],
                          dtype=np.uint64))
    return s[0]


def _uniform53(seed: int, stream: int, start: int, n: int) -> np.ndarray:
    """n float64 uniforms in [0, 1) from counters start..start+n-1."""
    base = _base(seed, stream)
    with np.errstate(over="ignore"):
        ctr = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = _mix(base + ctr * _GOLDEN)
    return (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)


def normal(seed: int, stream: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        m = min(_CHUNK, n - s)
        u = _uniform53(seed, stream, 2 * s, 2 * m)
        u1 = 1.0 - u[0::2]                      # (0, 1]
        u2 = u[1::2]
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * math.pi * u2)
        out[s:s + m] = (mean + std * z).astype(np.float32)
    return out.reshape(shape)


def uniform(seed: int, stream: int, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape)) if len(shape) else 1
    out = np.empty(n, dtype=np.float32)
    for s in range(0, n, _CHUNK):
        m = min(_CHUNK, n - s)
        out[s:s + m] = (lo + (hi - lo) * _uniform53(seed, stream, s, m)).astype(np.float32)
    return out.reshape(shape)


# stream ids (stable: never renumber)
S_WQKV, S_WZ, S_WB, S_WA, S_WOUT, S_CONV, S_ALOG, S_DT, S_GNORM = range(1, 10)
S_X, S_QKV, S_Z, S_A, S_B, S_STATE, S_CONVST = range(20, 27)
S_AQ, S_AK, S_AV, S_AO, S_AQN, S_AKN, S_AX, S_KPRE, S_VPRE = range(40, 49)


def layer_weights(d, seed: int = 0, gnorm_std: float = 0.0, proj_std: float = 0.02,
                  projections: bool = True) -> dict:
    """Random GDN layer weights for dims ``d`` (attributes kh, vh, kd, vd, K, hidden)."""
    conv_dim = 2 * d.kh * d.kd + d.vh * d.vd
    vdim = d.vh * d.vd
    w = {
        "conv_w": normal(seed, S_CONV, (conv_dim, d.K), 0.0, 0.1),
        "A_log": uniform(seed, S_ALOG, (d.vh,), 0.0, math.log(16.0)),
        "dt_bias": normal(seed, S_DT, (d.vh,), 0.0, 0.1),
        "gnorm": (np.ones(d.vd, np.float32) if gnorm_std == 0.0
                  else normal(seed, S_GNORM, (d.vd,), 1.0, gnorm_std)),
    }
    if projections:
        D = d.hidden
        w.update({
            "W_qkv": normal(seed, S_WQKV, (conv_dim, D), 0.0, proj_std),
            "W_z": normal(seed, S_WZ, (vdim, D), 0.0, proj_std),
            "W_b": normal(seed, S_WB, (d.vh, D), 0.0, proj_std),
            "W_a": normal(seed, S_WA, (d.vh, D), 0.0, proj_std),
            "W_out": normal(seed, S_WOUT, (D, vdim), 0.0, proj_std),
        })
    return w


def core_inputs(d, T: int, seed: int = 0, a_mean: float = 0.0, B: int | None = None) -> dict:
    """Pre-projected core inputs: mixed_qkv, z, a, b ~ N(0,1) (a ~ N(a_mean, 1)).

    Shapes are [T][...] (or [B][T][...] when B is given)."""
    conv_dim = 2 * d.kh * d.kd + d.vh * d.vd
    vdim = d.vh * d.vd
    lead = (T,) if B is None else (B, T)
    return {
        "qkv": normal(seed, S_QKV, lead + (conv_dim,)),
        "z": normal(seed, S_Z, lead + (vdim,)),
        "a": normal(seed, S_A, lead + (d.vh,), a_mean, 1.0),
        "b": normal(seed, S_B, lead + (d.vh,)),
    }


def states(d, seed: int = 0, s_std: float = 0.05, conv_std: float = 1.0, B: int | None = None):
    """Nonzero (conv_st [conv_dim][K-1], S [vh][kd][vd]) initial states."""
    conv_dim = 2 * d.kh * d.kd + d.vh * d.vd
    lead = () if B is None else (B,)
    S = normal(seed, S_STATE, lead + (d.vh, d.kd, d.vd), 0.0, s_std)
    conv = normal(seed, S_CONVST, lead + (conv_dim, d.K - 1), 0.0, conv_std)
    return conv, S


def attn_weights(D: int, H: int, KV: int, hd: int, seed: int = 0, proj_std: float = 0.02,
                 norm_std: float = 0.1) -> dict:
    """Random gated-attention weights (the omh_attn_weights names): q_proj
    [2*H*hd][D] (per head [hd q | hd gate]), k_proj / v_proj [KV*hd][D],
    o_proj [D][H*hd], q_norm / k_norm [hd] (used as 1 + w)."""
    return {"W_q": normal(seed, S_AQ, (2 * H * hd, D), 0.0, proj_std),
            "W_k": normal(seed, S_AK, (KV * hd, D), 0.0, proj_std),
            "W_v": normal(seed, S_AV, (KV * hd, D), 0.0, proj_std),
            "W_o": normal(seed, S_AO, (D, H * hd), 0.0, proj_std),
            "q_norm": normal(seed, S_AQN, (hd,), 0.0, norm_std),
            "k_norm": normal(seed, S_AKN, (hd,), 0.0, norm_std)}


def attn_inputs(D: int, KV: int, hd: int, pos0: int, T: int, seed: int = 0):
    """x [T][D] ~ N(0,1) and a prefilled cache Kpre / Vpre [pos0][KV][hd]:
    keys of unit RMS (as RMSNorm leaves them), values ~ N(0,1)."""
    return (normal(seed, S_AX, (T, D)), normal(seed, S_KPRE, (pos0, KV, hd)),
            normal(seed, S_VPRE, (pos0, KV, hd)))
