"""ctypes front-end to libom_hip.so (the C-ABI of include/om_hip.h).

This is the Python mirror of the engine-side calls for the GDN path: a
``GdnLayer`` owns one layer id of the library (weights uploaded once, state
for ``max_seqs`` sequences kept on the device) and exposes the same entry
points the C engine uses.  There is no CPU fallback here: if the library or
the GPU is missing, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .dims import GdnDims

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libom_hip.so")

OMH_OK, OMH_ERR_ALLOC, OMH_ERR_ARG, OMH_ERR_SHAPE, OMH_ERR_DEVICE = 0, -1, -2, -3, -4

# every entry point include/om_hip.h declares
EXPORTS = (
    "omh_init", "omh_last_error", "omh_gdn_layer_init", "omh_gdn_layer_free",
    "omh_gdn_state_reset", "omh_gdn_state_get", "omh_gdn_state_set",
    "omh_gdn_decode", "omh_gdn_prefill", "omh_gdn_decode_core", "omh_gdn_prefill_core",
    "omh_gdn_decode_core_dev", "omh_gdn_prefill_core_dev", "omh_gdn_decode_dev",
    "omh_gdn_prefill_dev", "omh_sync",
    "omh_attn_layer_init", "omh_attn_layer_free", "omh_attn_forward", "omh_attn_forward_dev",
    "omh_gdn_state_copy", "omh_gdn_state_copy_dev", "omh_attn_cache_get", "omh_attn_cache_set",
    "omh_gdn_decode_noalloc_dev", "omh_gdn_decode_core_seq_dev",
)


class OmhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"om_hip error {code}: {msg}")
        self.code = code


class _Dims(C.Structure):
    _fields_ = [("kh", C.c_int), ("vh", C.c_int), ("kd", C.c_int), ("vd", C.c_int),
                ("conv_k", C.c_int), ("hidden", C.c_int), ("eps", C.c_float)]


_WFIELDS = ("W_qkv", "W_z", "W_b", "W_a", "W_out", "Q_qkv", "Q_z", "Q_out",
            "S_qkv", "S_z", "S_out", "conv_w", "A_log", "dt_bias", "gnorm")


class _Weights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _WFIELDS]


class _AttnDims(C.Structure):
    _fields_ = [("hidden", C.c_int), ("n_heads", C.c_int), ("n_kv", C.c_int), ("head_dim", C.c_int),
                ("rot_dim", C.c_int), ("theta", C.c_float), ("eps", C.c_float), ("max_t", C.c_int)]


_AFIELDS = ("W_q", "W_k", "W_v", "W_o", "Q_q", "Q_k", "Q_v", "Q_o",
            "S_q", "S_k", "S_v", "S_o", "q_norm", "k_norm")


class _AttnWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _AFIELDS]


_LIB = None


def lib() -> C.CDLL:
    """Load libom_hip.so; raises if it was not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -c 'import __graft_entry__ as g; g.build()'`")
        L = C.CDLL(LIB_PATH)
        vp, ip, i = C.c_void_p, C.c_int, C.c_int
        L.omh_init.restype = ip
        L.omh_last_error.restype = C.c_char_p
        L.omh_gdn_layer_init.argtypes = [i, C.POINTER(_Dims), C.POINTER(_Weights), i]
        L.omh_gdn_layer_free.argtypes = [i]
        L.omh_gdn_state_reset.argtypes = [i, i]
        L.omh_gdn_state_get.argtypes = [i, i, vp, vp]
        L.omh_gdn_state_set.argtypes = [i, i, vp, vp]
        L.omh_gdn_decode.argtypes = [i, i, vp, vp]
        L.omh_gdn_prefill.argtypes = [i, i, i, vp, vp]
        L.omh_gdn_decode_core.argtypes = [i, i, vp, vp, vp, vp, vp]
        L.omh_gdn_prefill_core.argtypes = [i, i, i, vp, vp, vp, vp, vp]
        L.omh_gdn_decode_core_dev.argtypes = [i, C.POINTER(C.c_int), i, vp, vp, vp, vp, vp, vp]
        L.omh_gdn_decode_core_seq_dev.argtypes = [i, C.POINTER(C.c_int), i, i, vp, vp, vp, vp, vp, vp]
        L.omh_gdn_prefill_core_dev.argtypes = [i, i, i, vp, vp, vp, vp, vp, vp]
        L.omh_gdn_decode_dev.argtypes = [i, i, vp, vp, vp]
        L.omh_gdn_prefill_dev.argtypes = [i, i, i, vp, vp, vp]
        L.omh_gdn_decode_noalloc_dev.argtypes = [i, i, vp, vp, vp]
        L.omh_sync.argtypes = [vp]
        L.omh_gdn_state_copy.argtypes = [i, C.POINTER(C.c_int), i, i]
        L.omh_gdn_state_copy_dev.argtypes = [i, C.POINTER(C.c_int), i, i, vp]
        L.omh_attn_layer_init.argtypes = [i, C.POINTER(_AttnDims), C.POINTER(_AttnWeights), i]
        L.omh_attn_layer_free.argtypes = [i]
        L.omh_attn_forward.argtypes = [i, i, i, i, vp, vp]
        L.omh_attn_forward_dev.argtypes = [i, i, i, i, vp, vp, vp]
        L.omh_attn_cache_get.argtypes = [i, i, i, i, vp, vp, i]
        L.omh_attn_cache_set.argtypes = [i, i, i, i, vp, vp, i]
        _LIB = L
    return _LIB


def available() -> bool:
    return bool(lib().omh_init())


def last_error() -> str:
    return lib().omh_last_error().decode()


def check(rc: int) -> None:
    if rc != OMH_OK:
        raise OmhError(rc, last_error())


def require_gpu() -> None:
    if not available():
        raise OmhError(OMH_ERR_DEVICE, last_error())


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a) -> int | None:
    if a is None:
        return None
    if isinstance(a, int):                     # raw device address
        return a
    if hasattr(a, "data_ptr"):                 # torch tensor (device memory)
        return a.data_ptr()
    return a.ctypes.data


def quantize_rows(W: np.ndarray):
    """Per-row absmax int8 quantisation with the engine's rule
    (engines/qwen.c:124-138): s = max|w|/127 floored at 1e-8, q = rint(w/s)
    (ties to even, as lrintf) clamped to [-128, 127].  Host-side load step."""
    W = _f32(W)
    am = np.abs(W).max(axis=1)
    s = (am / np.float32(127.0)).astype(np.float32)
    s = np.where(s < np.float32(1e-8), np.float32(1e-8), s).astype(np.float32)
    q = np.clip(np.rint(W / s[:, None]), -128, 127).astype(np.int8)
    return q, s


class GdnLayer:
    """One GDN layer held by the library under id ``li``.

    ``weights`` holds numpy arrays named as in omh_gdn_weights (W_qkv, ...,
    conv_w, A_log, dt_bias, gnorm).  With ``int8=True`` the qkv, z and out
    projections are quantised per row here (the engine's load-time step,
    engines/qwen.c:269-274) and uploaded as int8 twins."""

    def __init__(self, li: int, dims: GdnDims, weights: dict, max_seqs: int = 1, int8: bool = False):
        require_gpu()
        self.li, self.dims, self.max_seqs = li, dims, max_seqs
        keep = {k: _f32(v) for k, v in weights.items() if not k.startswith(("Q_", "S_"))}
        keep.update({k: v for k, v in weights.items() if k.startswith(("Q_", "S_"))})
        if int8 and "W_qkv" in keep:
            for nm in ("qkv", "z", "out"):
                keep["Q_" + nm], keep["S_" + nm] = quantize_rows(keep["W_" + nm])
        self._keep = keep
        w = _Weights(**{k: (_ptr(keep[k]) if k in keep else None) for k in _WFIELDS})
        d = _Dims(dims.kh, dims.vh, dims.kd, dims.vd, dims.K, dims.hidden, dims.eps)
        check(lib().omh_gdn_layer_init(li, C.byref(d), C.byref(w), max_seqs))
        self.has_proj = "W_qkv" in keep

    def free(self) -> None:
        check(lib().omh_gdn_layer_free(self.li))

    def reset(self, seq: int = -1) -> None:
        check(lib().omh_gdn_state_reset(self.li, seq))

    def get_state(self, seq: int = 0):
        d = self.dims
        conv = np.empty((d.conv_dim, d.K - 1), np.float32)
        S = np.empty((d.vh, d.kd, d.vd), np.float32)
        check(lib().omh_gdn_state_get(self.li, seq, _ptr(conv), _ptr(S)))
        return conv, S

    def set_state(self, seq: int, conv=None, S=None) -> None:
        conv = None if conv is None else _f32(conv)
        S = None if S is None else _f32(S)
        check(lib().omh_gdn_state_set(self.li, seq, _ptr(conv), _ptr(S)))

    # ---- host-pointer entry points ----
    def copy_state(self, src_seq: int, dst_seq: int) -> None:
        """Device-side copy of one sequence's whole state over another's
        (snapshot before speculative tokens, rollback after a rejection)."""
        state_copy([self.li], src_seq, dst_seq)

    def decode(self, x: np.ndarray) -> np.ndarray:
        x = _f32(x)
        B = x.shape[0]
        out = np.empty((B, self.dims.hidden), np.float32)
        check(lib().omh_gdn_decode(self.li, B, _ptr(x), _ptr(out)))
        return out

    def decode_core(self, qkv, z, a, b) -> np.ndarray:
        qkv, z, a, b = _f32(qkv), _f32(z), _f32(a), _f32(b)
        B = qkv.shape[0]
        core = np.empty((B, self.dims.val_dim), np.float32)
        check(lib().omh_gdn_decode_core(self.li, B, _ptr(qkv), _ptr(z), _ptr(a), _ptr(b), _ptr(core)))
        return core

    def prefill(self, seq: int, x: np.ndarray) -> np.ndarray:
        x = _f32(x)
        T = x.shape[0]
        out = np.empty((T, self.dims.hidden), np.float32)
        check(lib().omh_gdn_prefill(self.li, seq, T, _ptr(x), _ptr(out)))
        return out

    def prefill_core(self, seq: int, qkv, z, a, b) -> np.ndarray:
        qkv, z, a, b = _f32(qkv), _f32(z), _f32(a), _f32(b)
        T = qkv.shape[0]
        core = np.empty((T, self.dims.val_dim), np.float32)
        check(lib().omh_gdn_prefill_core(self.li, seq, T, _ptr(qkv), _ptr(z), _ptr(a), _ptr(b),
                                         _ptr(core)))
        return core


# ---- device-pointer entry points (torch tensors, caller's stream) ----

def _stream(stream) -> int | None:
    if stream is None:
        return None
    return getattr(stream, "cuda_stream", stream)


def decode_core_dev(lis, B: int, qkv, z, a, b, core, stream=None) -> None:
    arr = (C.c_int * len(lis))(*lis)
    check(lib().omh_gdn_decode_core_dev(len(lis), arr, B, _ptr(qkv), _ptr(z), _ptr(a), _ptr(b),
                                        _ptr(core), _stream(stream)))


def decode_core_seq_dev(lis, seq0: int, B: int, qkv, z, a, b, core, stream=None) -> None:
    """decode_core_dev for sequences seq0 .. seq0+B-1 of every listed layer."""
    arr = (C.c_int * len(lis))(*lis)
    check(lib().omh_gdn_decode_core_seq_dev(len(lis), arr, seq0, B, _ptr(qkv), _ptr(z), _ptr(a), _ptr(b),
                                            _ptr(core), _stream(stream)))


def prefill_core_dev(li: int, seq: int, T: int, qkv, z, a, b, core, stream=None) -> None:
    check(lib().omh_gdn_prefill_core_dev(li, seq, T, _ptr(qkv), _ptr(z), _ptr(a), _ptr(b),
                                         _ptr(core), _stream(stream)))


def decode_dev(li: int, B: int, x, out, stream=None) -> None:
    check(lib().omh_gdn_decode_dev(li, B, _ptr(x), _ptr(out), _stream(stream)))


def decode_noalloc_dev(li: int, B: int, x, out, stream=None) -> None:
    """decode_dev with the library's static scratch: allocates nothing."""
    check(lib().omh_gdn_decode_noalloc_dev(li, B, _ptr(x), _ptr(out), _stream(stream)))


def prefill_dev(li: int, seq: int, T: int, x, out, stream=None) -> None:
    check(lib().omh_gdn_prefill_dev(li, seq, T, _ptr(x), _ptr(out), _stream(stream)))


def sync(stream=None) -> None:
    check(lib().omh_sync(_stream(stream)))


class AttnLayer:
    """One gated full-attention layer (engines/qwen.c:366-425) held by the
    library under attention id ``li`` (a namespace apart from the GDN ids),
    with a K/V cache of ``max_t`` positions for each of ``max_seqs``
    sequences.

    ``weights`` holds numpy arrays named as in omh_attn_weights (W_q, W_k,
    W_v, W_o, q_norm, k_norm); with ``int8=True`` the four projections are
    quantised per row here (the engine's load-time step, qwen.c:252-255)."""

    def __init__(self, li: int, hidden: int, n_heads: int, n_kv: int, head_dim: int, rot_dim: int,
                 theta: float, eps: float, max_t: int, weights: dict, max_seqs: int = 1, int8: bool = False):
        require_gpu()
        self.li, self.hidden = li, hidden
        self.n_kv, self.head_dim = n_kv, head_dim
        keep = {k: (v if k.startswith(("Q_", "S_")) else _f32(v)) for k, v in weights.items()}
        if int8:
            for nm in ("q", "k", "v", "o"):
                keep["Q_" + nm], keep["S_" + nm] = quantize_rows(keep.pop("W_" + nm))
        self._keep = keep
        w = _AttnWeights(**{k: (_ptr(keep[k]) if k in keep else None) for k in _AFIELDS})
        d = _AttnDims(hidden, n_heads, n_kv, head_dim, rot_dim, theta, eps, max_t)
        check(lib().omh_attn_layer_init(li, C.byref(d), C.byref(w), max_seqs))

    def free(self) -> None:
        check(lib().omh_attn_layer_free(self.li))

    def cache_get(self, seq: int, t0: int, n: int, ld_t: int | None = None):
        """Cache rows t0..t0+n-1 as the engine holds them: K, V [KV][ld_t][hd]
        (rows outside t0..t0+n-1 are zero)."""
        ld_t = ld_t or t0 + n
        K = np.zeros((self.n_kv, ld_t, self.head_dim), np.float32)
        V = np.zeros_like(K)
        check(lib().omh_attn_cache_get(self.li, seq, t0, n, _ptr(K), _ptr(V), ld_t))
        return K, V

    def cache_set(self, seq: int, t0: int, n: int, K: np.ndarray, V: np.ndarray) -> None:
        """Rows t0..t0+n-1 of host K, V [KV][ld_t][hd] into the device cache."""
        K, V = _f32(K), _f32(V)
        check(lib().omh_attn_cache_set(self.li, seq, t0, n, _ptr(K), _ptr(V), K.shape[1]))

    def forward(self, seq: int, pos: int, x: np.ndarray) -> np.ndarray:
        """x [T][hidden] at positions pos .. pos+T-1 -> [T][hidden]."""
        x = _f32(x)
        out = np.empty_like(x)
        check(lib().omh_attn_forward(self.li, seq, pos, x.shape[0], _ptr(x), _ptr(out)))
        return out


def attn_forward_dev(li: int, seq: int, pos: int, T: int, x, out, stream=None) -> None:
    check(lib().omh_attn_forward_dev(li, seq, pos, T, _ptr(x), _ptr(out), _stream(stream)))


def state_copy(lis, src_seq: int, dst_seq: int) -> None:
    """Snapshot / rollback of one sequence's state across layers lis (one launch)."""
    arr = (C.c_int * len(lis))(*lis)
    check(lib().omh_gdn_state_copy(len(lis), arr, src_seq, dst_seq))


def state_copy_dev(lis, src_seq: int, dst_seq: int, stream=None) -> None:
    arr = (C.c_int * len(lis))(*lis)
    check(lib().omh_gdn_state_copy_dev(len(lis), arr, src_seq, dst_seq, _stream(stream)))
