"""Host restatement of the reference qwen engine around the GDN layers
(TEST INFRASTRUCTURE ONLY: the end-to-end gate's checker).

Everything except the Gated DeltaNet layers follows overhang
engines/qwen.c in float32 numpy:
  * zero-centred RMSNorm, mean of squares in double (qwen.c:148-152);
  * gated full attention: q_proj rows per head [hd q | hd gate], q/k
    RMSNorm, partial RoPE on the first rot = head_dim * partial_rotary_factor
    dims as two halves, KV cache, softmax, sigmoid output gate, o_proj
    (qwen.c:366-425);
  * MoE: sigmoid-gated shared expert plus softmax router -> top-k ->
    renormalised expert mix (qwen.c:461-505);
  * step(): residual stream, final norm, lm_head (qwen.c:507-528).

The GDN layers (qwen.c:301-364) come from a pluggable backend:
``OracleGdn`` (the C restatement in oracle/, CPU) or ``HipGdn``
(libom_hip.so through the C-ABI, GPU).  The fixture is the reference's
tiny model (oracle/qwen_tiny: model.safetensors, config.json) and its
ref_qwen.json, copied under tests/golden/qwen_tiny.
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
TINY_DIR = os.path.join(HERE, "golden", "qwen_tiny")

f32 = np.float32


def load_tiny(path: str = TINY_DIR):
    from safetensors.numpy import load_file
    cfg = json.load(open(os.path.join(path, "config.json")))
    cfg = cfg.get("text_config", cfg)
    W = load_file(os.path.join(path, "model.safetensors"))
    ref = json.load(open(os.path.join(path, "ref_qwen.json")))
    return cfg, {k: np.ascontiguousarray(v, dtype=f32) for k, v in W.items()}, ref


def rmsnorm(x, w, eps):
    """qwen.c:148-152: x * 1/sqrtf((float)(mean(x^2) in double) + eps) * (1 + w)."""
    ms = np.mean(np.asarray(x, np.float64) ** 2, axis=-1, keepdims=True)
    r = (f32(1.0) / np.sqrt((ms.astype(f32) + f32(eps)))).astype(f32)
    return (x * r * (f32(1.0) + w)).astype(f32)


def sigmoid(z):
    return (f32(1.0) / (f32(1.0) + np.exp(-z))).astype(f32)


def silu(z):
    return (z * sigmoid(z)).astype(f32)


def softmax(x):
    """qwen.c:164-168: exp in float, sum in double."""
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m).astype(f32)
    s = np.sum(np.asarray(e, np.float64), axis=-1, keepdims=True).astype(f32)
    return (e / s).astype(f32)


def gdn_dims(cfg):
    from overhang_amd.dims import GdnDims
    return GdnDims(kh=cfg["linear_num_key_heads"], vh=cfg["linear_num_value_heads"],
                   kd=cfg["linear_key_head_dim"], vd=cfg["linear_value_head_dim"],
                   K=cfg.get("linear_conv_kernel_dim", 4), hidden=cfg["hidden_size"],
                   eps=cfg.get("rms_norm_eps", 1e-6))


def gdn_weights(W, i, d):
    p = f"model.layers.{i}.linear_attn."
    conv_dim = 2 * d.kh * d.kd + d.vh * d.vd
    return {
        "W_qkv": W[p + "in_proj_qkv.weight"], "W_z": W[p + "in_proj_z.weight"],
        "W_b": W[p + "in_proj_b.weight"], "W_a": W[p + "in_proj_a.weight"],
        "W_out": W[p + "out_proj.weight"],
        "conv_w": np.ascontiguousarray(W[p + "conv1d.weight"].reshape(conv_dim, d.K)),
        "A_log": W[p + "A_log"], "dt_bias": W[p + "dt_bias"], "gnorm": W[p + "norm.weight"],
    }


class OracleGdn:
    """GDN layers through the C oracle (one sequence, state carried)."""

    def __init__(self, d, weights):
        import oracle
        self.oracle, self.d, self.w = oracle, d, weights
        self.conv = {i: np.zeros((d.conv_dim, d.K - 1), f32) for i in weights}
        self.S = {i: np.zeros((d.vh, d.kd, d.vd), f32) for i in weights}

    def run(self, i, x):                       # x [T][D] -> [T][D]
        out, self.conv[i], self.S[i] = self.oracle.layer_seq(self.d, self.w[i], x, self.conv[i], self.S[i])
        return out

    def close(self):
        pass


class HipGdn:
    """GDN layers on the GPU through libom_hip.so: one token per call
    (omh_gdn_decode) or T tokens at once (omh_gdn_prefill)."""

    def __init__(self, d, weights, first_li=900, batched=False):
        from overhang_amd import gdn
        self.L = {i: gdn.GdnLayer(first_li + i, d, w) for i, w in weights.items()}
        self.batched = batched

    def run(self, i, x):
        if x.shape[0] == 1 and not self.batched:
            return self.L[i].decode(x)
        return self.L[i].prefill(0, x)

    def close(self):
        for L in self.L.values():
            L.free()


_ATTN_W = ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm")


_LIBM = None


def rope_inv_freq(theta, rot):
    """powf(theta, -(float)(2j)/(float)rot) for j < rot/2 (qwen.c:391), through
    the C library's own powf: numpy's float32 power can differ from it by an
    ulp, which at positions in the thousands moves the rotation angle by
    ~1e-4 rad."""
    global _LIBM
    if _LIBM is None:
        _LIBM = ctypes.CDLL("libm.so.6")
        _LIBM.powf.restype = ctypes.c_float
        _LIBM.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return np.array([_LIBM.powf(f32(theta), f32(-f32(2 * j) / f32(rot))) for j in range(rot // 2)], f32)


def gated_attention(x, W, Kl, Vl, pos, H, KV, hd, rot, theta, eps):
    """The engine's attn_step (qwen.c:366-425) for T tokens x [T][D] at
    positions pos..pos+T-1, in float32: q/gate split per head (qwen.c:376-382),
    RMSNorm of q and k with (1 + w) (385-386), partial RoPE over the first rot
    dims as two halves (388-398), causal softmax attention over the cache
    (405-419), output gate and o_proj (421-422).  W maps q_proj, k_proj,
    v_proj, o_proj, q_norm, k_norm to arrays; Kl / Vl are the lists of
    [t][KV][hd] cache blocks, appended to here."""
    T = x.shape[0]
    qg = (x @ W["q_proj"].T).reshape(T, H, 2 * hd)
    q, gate = qg[:, :, :hd], qg[:, :, hd:].reshape(T, H * hd)
    k = (x @ W["k_proj"].T).reshape(T, KV, hd)
    v = (x @ W["v_proj"].T).reshape(T, KV, hd)
    q = rmsnorm(q, W["q_norm"], eps)
    k = rmsnorm(k, W["k_norm"], eps)
    half = rot // 2
    inv = rope_inv_freq(theta, rot)
    ps = np.arange(pos, pos + T, dtype=f32)[:, None]
    ang = (ps * inv[None, :]).astype(f32)
    cs, sn = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]

    def rope(vec):
        a0, b0 = vec[..., :half].copy(), vec[..., half:rot].copy()
        vec = vec.copy()
        vec[..., :half] = a0 * cs - b0 * sn
        vec[..., half:rot] = b0 * cs + a0 * sn
        return vec.astype(f32)

    q, k = rope(q), rope(k)
    Kl.append(k)
    Vl.append(v)
    Kc, Vc = np.concatenate(Kl), np.concatenate(Vl)                      # [pos+T][KV][hd]
    n = Kc.shape[0]
    grp = H // KV
    ctx = np.empty((T, H, hd), f32)
    scale = f32(1.0) / np.sqrt(f32(hd))
    for h in range(H):
        sc = (q[:, h, :] @ Kc[:, h // grp, :].T).astype(f32) * scale        # [T][n]
        mask = np.arange(n)[None, :] > (pos + np.arange(T))[:, None]
        sc[mask] = -np.inf
        ctx[:, h, :] = softmax(sc) @ Vc[:, h // grp, :]
    ctx = ctx.reshape(T, H * hd) * sigmoid(gate)
    return (ctx @ W["o_proj"].T).astype(f32)


class TinyQwen:
    """The reference engine's forward (qwen.c:507-528) with the GDN layers
    delegated to ``backend(d, {layer: weights})``."""

    def __init__(self, backend_cls, path: str = TINY_DIR, gpu_attn_li=None, **kw):
        self.cfg, self.W, self.ref = load_tiny(path)
        c = self.cfg
        self.D, self.eps = c["hidden_size"], c.get("rms_norm_eps", 1e-6)
        self.nl = c["num_hidden_layers"]
        self.full_every = c.get("full_attention_interval", 4)
        self.H, self.KV, self.hd = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        rp = c.get("rope_parameters", {})
        self.rot = int(self.hd * rp.get("partial_rotary_factor", c.get("partial_rotary_factor", 1.0)))
        self.theta = float(rp.get("rope_theta", 1e7))
        self.E, self.topk = c["num_experts"], c["num_experts_per_tok"]
        self.d = gdn_dims(c)
        self.is_full = [((i + 1) % self.full_every) == 0 for i in range(self.nl)]
        gw = {i: gdn_weights(self.W, i, self.d) for i in range(self.nl) if not self.is_full[i]}
        self.gdn = backend_cls(self.d, gw, **kw)
        self.K = {i: [] for i in range(self.nl) if self.is_full[i]}
        self.V = {i: [] for i in range(self.nl) if self.is_full[i]}
        self.pos = 0
        self.attn_gpu = None
        if gpu_attn_li is not None:                 # attention layers on libom_hip.so too
            from overhang_amd import gdn
            self.attn_gpu = {}
            for i in self.K:
                p = f"model.layers.{i}.self_attn."
                w = {"W_q": self.W[p + "q_proj.weight"], "W_k": self.W[p + "k_proj.weight"],
                     "W_v": self.W[p + "v_proj.weight"], "W_o": self.W[p + "o_proj.weight"],
                     "q_norm": self.W[p + "q_norm.weight"], "k_norm": self.W[p + "k_norm.weight"]}
                self.attn_gpu[i] = gdn.AttnLayer(gpu_attn_li + i, self.D, self.H, self.KV, self.hd, self.rot,
                                                 self.theta, self.eps, 64, w)
        self.lm_head = self.W.get("lm_head.weight", self.W["model.embed_tokens.weight"])

    def close(self):
        self.gdn.close()
        for L in (self.attn_gpu or {}).values():
            L.free()

    # -- gated full attention over T new tokens at positions pos..pos+T-1 (qwen.c:366-425)
    def attn(self, i, x):
        if self.attn_gpu is not None:
            return self.attn_gpu[i].forward(0, self.pos, x)
        p = f"model.layers.{i}.self_attn."
        return gated_attention(x, {n: self.W[p + n + ".weight"] for n in _ATTN_W}, self.K[i], self.V[i],
                               self.pos, self.H, self.KV, self.hd, self.rot, self.theta, self.eps)

    # -- MoE (qwen.c:461-505)
    def moe(self, i, x):
        p = f"model.layers.{i}.mlp."
        g = x @ self.W[p + "shared_expert.gate_proj.weight"].T
        u = x @ self.W[p + "shared_expert.up_proj.weight"].T
        out = (silu(g) * u) @ self.W[p + "shared_expert.down_proj.weight"].T
        sg = sigmoid(x @ self.W[p + "shared_expert_gate.weight"].T)          # [T][1]
        out = (out * sg).astype(f32)
        pr = softmax((x @ self.W[p + "gate.weight"].T).astype(f32))          # [T][E]
        for t in range(x.shape[0]):
            idx = []
            for _ in range(self.topk):                                       # first maximum, as qwen.c:482-489
                cand = [e for e in range(self.E) if e not in idx]
                idx.append(max(cand, key=lambda e: (pr[t, e], -e)))
            val = pr[t, idx]
            val = (val / val.sum(dtype=f32)).astype(f32)
            for kk, e in enumerate(idx):
                q = f"{p}experts.{e}."
                ge = x[t] @ self.W[q + "gate_proj.weight"].T
                ue = x[t] @ self.W[q + "up_proj.weight"].T
                hh = (silu(ge) * ue) @ self.W[q + "down_proj.weight"].T
                out[t] += val[kk] * hh
        return out.astype(f32)

    def forward(self, ids):
        """T tokens at positions pos..pos+T-1; returns logits [T][vocab]."""
        x = self.W["model.embed_tokens.weight"][np.asarray(ids)].astype(f32)
        for i in range(self.nl):
            nrm = rmsnorm(x, self.W[f"model.layers.{i}.input_layernorm.weight"], self.eps)
            if self.is_full[i]:
                x = x + self.attn(i, nrm)
            else:
                x = x + self.gdn.run(i, np.ascontiguousarray(nrm))
            nrm = rmsnorm(x, self.W[f"model.layers.{i}.post_attention_layernorm.weight"], self.eps)
            x = (x + self.moe(i, nrm)).astype(f32)
        self.pos += len(ids)
        x = rmsnorm(x, self.W["model.norm.weight"], self.eps)
        return (x @ self.lm_head.T).astype(f32)


def greedy(model: TinyQwen):
    """The reference's validation main (qwen.c:621-658): prompt token by
    token, then greedy generation; returns (generated ids, expected ids)."""
    ref = model.ref
    prompt, full = ref["prompt_ids"], ref["full_ids"]
    logit = None
    for t in prompt:
        logit = model.forward([t])[0]
    out = []
    for i in range(len(full) - len(prompt)):
        best = int(np.argmax(logit))
        out.append(best)
        if i < len(full) - len(prompt) - 1:
            logit = model.forward([best])[0]
    return out, list(full[len(prompt):])


def teacher_forced(model: TinyQwen):
    """Teacher-forced argmax over full_ids in one batched forward (every
    layer sees all positions at once; the GDN layers prefill).  The
    reference records this from transformers' chunked path
    (make_qwen_oracle.py:68-69) as tf_argmax."""
    logits = model.forward(list(model.ref["full_ids"]))
    return [int(v) for v in np.argmax(logits, axis=-1)], list(model.ref["tf_argmax"])
