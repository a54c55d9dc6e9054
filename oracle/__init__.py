"""ctypes front-end to the CPU checkers (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package.  It wraps

* ``liboracle.so``  — gdn_oracle.c, the C restatement of the reference GDN
  (overhang engines/qwen.c:70-77, 116-138, 153-160, 301-364) plus a chunked
  WY/UT restatement (transformers modeling_qwen3_5_moe.py:250-328);
* ``_ref/libqwen_ref.so`` — the reference engine's own code compiled from the
  reference sources (present only where they were available at build time).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None
_REF = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")


class _Dims(C.Structure):
    _fields_ = [("kh", C.c_int), ("vh", C.c_int), ("kd", C.c_int), ("vd", C.c_int),
                ("K", C.c_int), ("hidden", C.c_int), ("eps", C.c_float)]


class _LayerW(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "W_qkv", "W_z", "W_b", "W_a", "W_out", "Q_qkv", "Q_z", "Q_out",
        "S_qkv", "S_z", "S_out", "conv_w", "A_log", "dt_bias", "gnorm")]


def build(ref: bool = True) -> None:
    """Compile liboracle.so (and _ref when the reference sources exist)."""
    subprocess.run(["make", "-s", "-C", HERE, "all" if ref else os.path.join(HERE, "liboracle.so")],
                   check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            build(ref=False)
        L = C.CDLL(path)
        L.gdno_matvec.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int]
        L.gdno_quantize_rows.argtypes = [_f32p, _i8p, _f32p, C.c_int, C.c_int]
        L.gdno_matmul_q.argtypes = [_f32p, _f32p, _i8p, _f32p, C.c_int, C.c_int]
        core_args = [C.POINTER(_Dims), _f32p, _f32p, _f32p, _f32p]
        L.gdno_core_seq.argtypes = core_args + [C.c_int, _f32p, _f32p, _f32p, _f32p,
                                                _f32p, _f32p, _f32p]
        L.gdno_layer_seq.argtypes = [C.POINTER(_Dims), C.POINTER(_LayerW), C.c_int, C.c_int,
                                     _f32p, _f32p, _f32p, _f32p]
        L.gdno_chunked.argtypes = [C.c_int] * 6 + [_f32p] * 7
        L.gdno_threads.restype = C.c_int
        _LIB = L
    return _LIB


def ref_lib():
    """The compiled reference checker, or None where it was not built."""
    global _REF
    if _REF is None:
        path = os.path.join(HERE, "_ref", "libqwen_ref.so")
        if not os.path.exists(path):
            return None
        L = C.CDLL(path)
        L.ref_gdn_layer_run.argtypes = ([C.c_int] * 6 + [C.c_float, C.c_int] + [_f32p] * 9
                                        + [C.c_int, _f32p, _f32p, _f32p, _f32p])
        L.ref_quantize_rows.argtypes = [_f32p, _i8p, _f32p, C.c_int, C.c_int]
        L.ref_matmul_q.argtypes = [_f32p, _f32p, _i8p, _f32p, C.c_int, C.c_int]
        L.ref_matvec.argtypes = [_f32p, _f32p, _f32p, C.c_int, C.c_int]
        L.ref_layer_open.argtypes = [C.c_int] * 6 + [C.c_float, C.c_int] + [_f32p] * 9
        L.ref_layer_steps.argtypes = [C.c_int, _f32p, C.c_void_p]
        L.ref_layer_close.argtypes = []
        L.ref_attn_run.argtypes = ([C.c_int] * 5 + [C.c_float, C.c_float, C.c_int] + [_f32p] * 6
                                   + [C.c_int, _f32p, _f32p, C.c_int, _f32p, _f32p, _f32p, _f32p])
        _REF = L
    return _REF


def _c(a, dt=np.float32):
    return np.ascontiguousarray(a, dtype=dt)


def _dims(d) -> _Dims:
    return _Dims(d.kh, d.vh, d.kd, d.vd, d.K, getattr(d, "hidden", 0), d.eps)


def threads() -> int:
    return lib().gdno_threads()


def matvec(x, W):
    O, I = W.shape
    y = np.empty(O, np.float32)
    lib().gdno_matvec(y, _c(x), _c(W), I, O)
    return y


def quantize_rows(W):
    O, I = W.shape
    q = np.empty((O, I), np.int8)
    s = np.empty(O, np.float32)
    lib().gdno_quantize_rows(_c(W), q, s, O, I)
    return q, s


def matmul_q(x, q, s):
    O, I = q.shape
    y = np.empty(O, np.float32)
    lib().gdno_matmul_q(y, _c(x), _c(q, np.int8), _c(s), I, O)
    return y


def core_seq(d, w, qkv, z, a, b, conv_st, S):
    """T tokens of the GDN core; returns (core [T][vh*vd], conv_st', S')."""
    qkv = _c(qkv)
    T = qkv.shape[0]
    conv_st = _c(conv_st).copy()
    S = _c(S).copy()
    core = np.empty((T, d.vh * d.vd), np.float32)
    dd = _dims(d)
    lib().gdno_core_seq(C.byref(dd), _c(w["conv_w"]), _c(w["A_log"]), _c(w["dt_bias"]),
                        _c(w["gnorm"]), T, qkv, _c(z), _c(a), _c(b), conv_st, S, core)
    return core, conv_st, S


def layer_seq(d, w, x, conv_st, S, int8: bool = False):
    """T tokens through the whole GDN layer; returns (out [T][D], conv_st', S').

    In int8 mode the int8 twins are made here with the restated quantiser, as
    the reference does at load (qwen.c:269-274)."""
    x = _c(x)
    T = x.shape[0]
    conv_st = _c(conv_st).copy()
    S = _c(S).copy()
    out = np.empty((T, d.hidden), np.float32)
    keep = {k: _c(v) for k, v in w.items()}
    if int8:
        for nm in ("qkv", "z", "out"):
            q, s = quantize_rows(keep["W_" + nm])
            keep["Q_" + nm], keep["S_" + nm] = q, s
    lw = _LayerW(**{k: (keep[k].ctypes.data if k in keep else None) for k, _ in _LayerW._fields_})
    dd = _dims(d)
    lib().gdno_layer_seq(C.byref(dd), C.byref(lw), int(int8), T, x, out, conv_st, S)
    return out, conv_st, S


def chunked(d, q, k, v, g, beta, S, C_: int = 64):
    """Chunked WY/UT restatement on normalised inputs (q,k [T][kh][kd], v [T][vh][vd],
    g, beta [T][vh]); returns (o [T][vh][vd], S')."""
    q = _c(q)
    T = q.shape[0]
    S = _c(S).copy()
    o = np.empty((T, d.vh, d.vd), np.float32)
    lib().gdno_chunked(d.kh, d.vh, d.kd, d.vd, T, C_, q, _c(k), _c(v), _c(g), _c(beta), S, o)
    return o, S


# ---- the compiled reference (checker of the checker) ----

def ref_layer_seq(d, w, x, conv_st, S, int8: bool = False):
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref not built (reference sources absent at build time)")
    x = _c(x)
    T = x.shape[0]
    conv_st = _c(conv_st).copy()
    S = _c(S).copy()
    out = np.empty((T, d.hidden), np.float32)
    R.ref_gdn_layer_run(d.kh, d.vh, d.kd, d.vd, d.K, d.hidden, d.eps, int(int8),
                        _c(w["W_qkv"]), _c(w["W_z"]), _c(w["W_b"]), _c(w["W_a"]), _c(w["W_out"]),
                        _c(w["conv_w"]), _c(w["A_log"]), _c(w["dt_bias"]), _c(w["gnorm"]),
                        T, x, out, conv_st, S)
    return out, conv_st, S


def ref_quantize_rows(W):
    O, I = W.shape
    q = np.empty((O, I), np.int8)
    s = np.empty(O, np.float32)
    ref_lib().ref_quantize_rows(_c(W), q, s, O, I)
    return q, s


def ref_matmul_q(x, q, s):
    O, I = q.shape
    y = np.empty(O, np.float32)
    ref_lib().ref_matmul_q(y, _c(x), _c(q, np.int8), _c(s), I, O)
    return y


def ref_matvec(x, W):
    O, I = W.shape
    y = np.empty(O, np.float32)
    ref_lib().ref_matvec(y, _c(x), _c(W), I, O)
    return y


def ref_attn_run(w, H, KV, hd, rot, theta, eps, pos0, Kpre, Vpre, x, int8: bool = False):
    """T tokens through the reference attn_step (qwen.c:367-425) at positions
    pos0..pos0+T-1 over a cache prefilled with Kpre / Vpre [pos0][KV][hd];
    returns (out [T][D], K rows written [T][KV][hd], V rows [T][KV][hd])."""
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref not built (reference sources absent at build time)")
    x = _c(x)
    T, D = x.shape
    out = np.empty((T, D), np.float32)
    Kn = np.empty((T, KV, hd), np.float32)
    Vn = np.empty((T, KV, hd), np.float32)
    if pos0 == 0:
        Kpre = np.zeros((1, KV, hd), np.float32)
        Vpre = Kpre
    rc = R.ref_attn_run(D, H, KV, hd, rot, theta, eps, int(int8), _c(w["W_q"]), _c(w["W_k"]),
                        _c(w["W_v"]), _c(w["W_o"]), _c(w["q_norm"]), _c(w["k_norm"]), pos0,
                        _c(Kpre), _c(Vpre), T, x, out, Kn, Vn)
    if rc != 0:
        raise ValueError(f"ref_attn_run: {rc}")
    return out, Kn, Vn


class RefLayer:
    """The reference's deltanet_step on one persistent synthetic layer (set up
    once: weights copied, int8 twins made with qw_make when int8), for timing
    it the way the engine calls it: one token per call, state carried."""

    def __init__(self, d, w, int8: bool = False):
        R = ref_lib()
        if R is None:
            raise RuntimeError("oracle/_ref not built (reference sources absent at build time)")
        self._keep = {k: _c(v) for k, v in w.items()}
        k = self._keep
        R.ref_layer_open(d.kh, d.vh, d.kd, d.vd, d.K, d.hidden, d.eps, int(int8), k["W_qkv"], k["W_z"],
                         k["W_b"], k["W_a"], k["W_out"], k["conv_w"], k["A_log"], k["dt_bias"], k["gnorm"])
        self.R, self.d = R, d

    def steps(self, x, out=None):
        x = _c(x)
        self.R.ref_layer_steps(x.shape[0], x, None if out is None else out.ctypes.data)

    def close(self):
        self.R.ref_layer_close()
