#!/usr/bin/env python3
"""GDN layer throughput on one MI355X, next to the CPU reference GDN.

Headline (the JSON line's `value`): decode of one token through the GDN core
of 30 layers at the Qwen3.6-35B-A3B GDN shape (kh=16, vh=32, kd=vd=128),
batch 1, pre-projected inputs (mixed_qkv, z, a, b), fp32 state.  The 30
layers' inputs are independent, so one launch serves all 30; every step uses
a different set of 30 layer states out of >1 GiB so the 256 MB Infinity
Cache cannot hold them (each step reads and writes 126 MB of state from HBM).

Also reported: the same step launched layer by layer (the order an engine
runs it), a batch sweep B=1..64 of one-layer launches, the chunked prefill
of T=4096 tokens at the same head shape (MFMA roofline), a 32768-token
prefill continuing from an 8192-token one (config 4), one decode step of the
whole block with int8 projections for 64 sequences (config 5, HBM roofline),
a device-to-device copy (the HBM bandwidth a plain copy reaches on this
box), and the CPU oracle (the reference GDN restated in C, OpenMP) on the
host cores.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--part all|decode|prefill|block]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "GDN tok/s: prefill T=4096 + decode B=1..64; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
FP32_MFMA_TFLOPS = 157.3
INT8_MFMA_TOPS = 5000.0
N_LAYERS = 30
ROTATE_BYTES = 1 << 30
# config 2's full compulsory bytes per layer and token at the 35B shape: state
# read + write 4,194,304, conv history read + write 196,608, conv weights
# 131,072, mixed_qkv / z / a / b in (49,408) and the core output out (16,384)
FULL_COMPULSORY_PER_LAYER = 4194304 + 196608 + 131072 + 49408 + 16384


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_layers(gdn, d, first_li, n, max_seqs, w, conv0, S0):
    lays = []
    for i in range(n):
        L = gdn.GdnLayer(first_li + i, d, w, max_seqs=max_seqs)
        for s in range(max_seqs):
            L.set_state(s, conv0, S0)
        lays.append(L)
    return lays


def time_launches(hip, st, fn, steps, warmup):
    """Run fn(k) for warmup + steps iterations on stream st.

    Throughput pass: `steps` back-to-back steps bracketed by device
    synchronisation, timed by one HIP event pair on st around the region.
    Duration pass: the same steps again, each between its own event pair on
    st (the per-launch kernel time the roofline uses).  Returns (elapsed s of
    the throughput region, per-step durations in s, host wall s)."""
    for k in range(warmup):
        fn(k)
    hip.device_synchronize()
    t0, t1 = hip.Event(), hip.Event()
    wall0 = time.perf_counter()
    t0.record(st)
    for k in range(steps):
        fn(warmup + k)
    t1.record(st)
    hip.device_synchronize()
    wall = time.perf_counter() - wall0
    el = t0.elapsed_ms(t1) / 1e3
    ev = [(hip.Event(), hip.Event()) for _ in range(steps)]
    for k in range(steps):
        ev[k][0].record(st)
        fn(warmup + steps + k)
        ev[k][1].record(st)
    hip.device_synchronize()
    durs = [a.elapsed_ms(b) / 1e3 for a, b in ev]
    return max(el, 1e-12), durs, wall


def bench_decode(hip, gdn, synth, steps, warmup, full=True, rotated=True):
    from overhang_amd.dims import Q35B
    d = Q35B
    per_layer = d.state_bytes + 4 * d.conv_dim * (d.K - 1)
    R = math.ceil(ROTATE_BYTES / (N_LAYERS * per_layer))
    log(f"decode: {N_LAYERS} layers x {R} sequence slots, {R * N_LAYERS * per_layer / 2**30:.2f} GiB of state")
    w = synth.layer_weights(d, 0, projections=False)
    conv0, S0 = synth.states(d, 0)
    # one model of 30 GDN layers (one set of weights per layer), R sequence
    # slots per layer; step k decodes slot k % R in every layer, so a slot's
    # state comes back every R steps, after more than 1 GiB of other states
    # has streamed through: the state reads and writes go to HBM
    lays = make_layers(gdn, d, 0, N_LAYERS, R, w, conv0, S0)
    inp = synth.core_inputs(d, N_LAYERS, 1)                # [30][...] = [nl][B=1][...]
    dev = {k: hip.Buffer.from_numpy(v) for k, v in inp.items()}
    row = {k: v.shape[1] * 4 for k, v in inp.items()}
    core = hip.Buffer(N_LAYERS * d.val_dim * 4)
    st = hip.Stream()
    lis = [L.li for L in lays]

    # the entry point bound once, its layer-id array and pointers built up
    # front, so the host issues a launch in a few microseconds and the
    # back-to-back launches keep the GPU busy
    import ctypes as C
    fn = gdn.lib().omh_gdn_decode_core_seq_dev
    arr = (C.c_int * N_LAYERS)(*lis)
    args = [gdn._ptr(dev[k]) for k in ("qkv", "z", "a", "b")] + [gdn._ptr(core), gdn._stream(st)]

    def step_fused(k):
        gdn.check(fn(N_LAYERS, arr, k % R, 1, *args))

    # (untimed warm-up: at least two passes over the slots, so every slot's
    # state has been through the kernel and the clocks have settled)
    el, durs, wall = time_launches(hip, st, step_fused, steps, max(warmup, 2 * R))
    # host time to issue one launch (no synchronisation inside the loop)
    hip.device_synchronize()
    h0 = time.perf_counter()
    for k in range(steps):
        step_fused(k)
    issue_us = 1e6 * (time.perf_counter() - h0) / steps
    hip.device_synchronize()
    alg_bytes = N_LAYERS * 2 * d.state_bytes                # state read + write, 30 layers
    # average launch duration = the timed region of back-to-back launches / launches
    kern = el / steps
    fused = {"tok_s": steps / el, "ms_per_step": 1e3 * el / steps, "kernel_us": 1e6 * kern,
             "kernel_us_isolated": 1e6 * statistics.mean(durs),
             "achieved_GBs": alg_bytes / kern / 1e9, "wall_s": wall, "host_issue_us_per_launch": issue_us}
    log(f"decode fused 30-layer launch: {fused['tok_s']:.0f} tok/s, kernel {fused['kernel_us']:.1f} us, "
        f"{fused['achieved_GBs']:.0f} GB/s, host issue {issue_us:.1f} us per launch")

    if rotated:
        fused["weights_rotated"] = bench_decode_weights_rotated(hip, gdn, synth, d, w, conv0, S0, inp, core, st,
                                                                steps, warmup)
    if not full:
        for L in lays:
            L.free()
        hip.device_synchronize()
        return fused, None, None, alg_bytes, R

    # engine order: one launch per layer (the order an engine issues them)
    def step_layers(k):
        for l in range(N_LAYERS):
            gdn.decode_core_seq_dev([lis[l]], k % R, 1, *(dev[nm].at(l * row[nm]) for nm in ("qkv", "z", "a", "b")),
                                    core.at(l * d.val_dim * 4), stream=st)

    n2 = max(steps // 2, 5)
    el2, durs2, _ = time_launches(hip, st, step_layers, n2, warmup)
    k2 = statistics.mean(durs2) / N_LAYERS
    engine = {"tok_s": n2 / el2, "ms_per_step": 1e3 * el2 / n2, "us_per_layer_incl_gaps": 1e6 * k2,
              "issue": "30 one-layer launches per token from Python (ctypes)"}
    log(f"decode engine order (30 launches/token, ctypes): {engine['tok_s']:.0f} tok/s")
    # the same 30 launches captured once in a HIP graph (two tokens per graph,
    # so every layer's ring epoch alternates as in eager use) and replayed
    graphs = [hip.Graph(st, lambda r=r: [step_layers(r), step_layers(r)]) for r in range(R)]
    def step_graph(k):
        graphs[k % R].launch()
    n3 = max(steps // 2, 5)
    el3, _, _ = time_launches(hip, st, step_graph, n3, warmup)
    engine_graph = {"tok_s": 2 * n3 / el3, "ms_per_step": 1e3 * el3 / (2 * n3),
                    "us_per_layer": 1e6 * el3 / (2 * n3 * N_LAYERS), "kernel_nodes_per_graph": graphs[0].nodes,
                    "issue": "30 one-layer launches per token, captured in a HIP graph (2 tokens per graph)"}
    log(f"decode engine order (graph): {engine_graph['tok_s']:.0f} tok/s, "
        f"{engine_graph['us_per_layer']:.2f} us per layer")
    for gr in graphs:
        gr.close()
    for L in lays:
        L.free()
    hip.device_synchronize()

    # batch sweep: one layer per launch, B sequences; every B rotates over
    # more than 1 GiB of distinct states (layers of max_seqs = B)
    sweep = []
    for B in (1, 2, 4, 8, 16, 32, 64):
        nrot = max(2, math.ceil(ROTATE_BYTES / (B * per_layer)))
        lays = make_layers(gdn, d, 1000, nrot, B, w, conv0, S0)
        inpB = synth.core_inputs(d, 1, 2, B=B)
        devB = {k: hip.Buffer.from_numpy(np.ascontiguousarray(v[:, 0])) for k, v in inpB.items()}
        coreB = hip.Buffer(B * d.val_dim * 4)

        def stepB(k, B=B):
            gdn.decode_core_dev([lays[k % nrot].li], B, devB["qkv"], devB["z"], devB["a"], devB["b"], coreB,
                                stream=st)
        nsteps = max(steps, 20)
        elB, dB, _ = time_launches(hip, st, stepB, nsteps, warmup)
        kb = elB / nsteps
        gbs = B * 2 * d.state_bytes / kb / 1e9
        sweep.append({"B": B, "kernel_us": 1e6 * kb, "achieved_GBs": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
                      "tok_s_30_layers": B / (N_LAYERS * kb), "rotation_bytes": nrot * B * per_layer})
        log(f"decode sweep B={B}: kernel {1e6 * kb:.1f} us, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}%), "
            f"rotating over {nrot * B * per_layer / 2**30:.2f} GiB")
        for L in lays:
            L.free()
        hip.device_synchronize()
    return fused, {"ctypes": engine, "graph": engine_graph}, sweep, alg_bytes, R


def bench_decode_weights_rotated(hip, gdn, synth, d, w, conv0, S0, inp, core, st, steps, warmup):
    """The headline launch with every rotation group a separate set of 30
    layers, each with its own copy of the conv weights as well as its own
    state (one slot each): the form earlier measurements of this build used.
    Every launch then also reads 30 x 128 KiB of conv weights from HBM."""
    import ctypes as C
    per_layer = d.state_bytes + 4 * d.conv_dim * (d.K - 1)
    R = math.ceil(ROTATE_BYTES / (N_LAYERS * per_layer))
    lays = make_layers(gdn, d, 3000, R * N_LAYERS, 1, w, conv0, S0)
    dev = {k: hip.Buffer.from_numpy(v) for k, v in inp.items()}
    fn = gdn.lib().omh_gdn_decode_core_dev
    arrs = [(C.c_int * N_LAYERS)(*[lays[r * N_LAYERS + l].li for l in range(N_LAYERS)]) for r in range(R)]
    args = [gdn._ptr(dev[k]) for k in ("qkv", "z", "a", "b")] + [gdn._ptr(core), gdn._stream(st)]
    el, _, _ = time_launches(hip, st, lambda k: gdn.check(fn(N_LAYERS, arrs[k % R], 1, *args)), steps, warmup)
    kern = el / steps
    gbs = N_LAYERS * 2 * d.state_bytes / kern / 1e9
    log(f"decode fused 30-layer launch, weights rotated with the states ({R} x 30 layers): kernel "
        f"{1e6 * kern:.1f} us, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}%)")
    for L in lays:
        L.free()
    hip.device_synchronize()
    return {"kernel_us": 1e6 * kern, "achieved_GBs": gbs, "frac_hbm": gbs / HBM_PEAK_GBS, "rotation_groups": R}


def quantized(w):
    """w plus its int8 twins (Q_*, S_* for qkv, z, out), made once with the
    engine's rule, so several layers can share one quantisation."""
    from overhang_amd import gdn
    w = dict(w)
    for nm in ("qkv", "z", "out"):
        w["Q_" + nm], w["S_" + nm] = gdn.quantize_rows(w["W_" + nm])
    return w


def bench_engine_block(hip, gdn, synth, steps, warmup):
    """The drop-in as an engine uses it at B = 1: one token through the whole
    GDN block (int8 in_proj -> core -> int8 out_proj) of each of 30 layers at
    the 35B shape, layer after layer, each layer's output the next one's
    input.  Every layer has its own weights and state (1.1 GB of weights in
    all, beyond the last-level cache).  Issued as omh_gdn_decode_noalloc_dev
    calls captured in a HIP graph (2 tokens per graph); also the latency of
    the host-pointer call omh_gdn_decode(li, 1, x, out), the exact
    deltanet_step replacement, with its copies."""
    from overhang_amd.dims import Q35B
    d = Q35B
    w = quantized(synth.layer_weights(d, 5))
    lays = [gdn.GdnLayer(2100 + i, d, w, max_seqs=1) for i in range(N_LAYERS)]
    bufs = [hip.Buffer.from_numpy(synth.normal(8, synth.S_X, (1, d.hidden), 0.0, 1.0))] + \
           [hip.Buffer(d.hidden * 4) for _ in range(N_LAYERS)]
    st = hip.Stream()

    def token():
        for l in range(N_LAYERS):
            gdn.decode_noalloc_dev(lays[l].li, 1, bufs[l], bufs[l + 1], stream=st)

    g = hip.Graph(st, lambda: [token(), token()])
    n = max(steps // 2, 5)
    el, _, _ = time_launches(hip, st, lambda k: g.launch(), n, warmup)
    per_tok = el / (2 * n)
    wbytes = block_bytes(d, 1) - 2 * (d.state_bytes + 4 * d.conv_dim * (d.K - 1)) - 2 * d.hidden * 4
    alg = N_LAYERS * block_bytes(d, 1)
    res = {"tok_s": 1 / per_tok, "us_per_token": 1e6 * per_tok, "us_per_layer": 1e6 * per_tok / N_LAYERS,
           "alg_bytes_per_token": alg, "achieved_GBs": alg / per_tok / 1e9,
           "frac_hbm": alg / per_tok / 1e9 / HBM_PEAK_GBS, "weight_bytes_per_layer": wbytes,
           "kernel_nodes_per_graph": g.nodes,
           "note": "30 GDN layers x whole block (int8 projections on the register GEMV, core), B=1, "
                   "dependent chain, HIP graph replay"}
    g.close()
    log(f"engine block chain (graph): {res['us_per_layer']:.2f} us/layer, {res['tok_s']:.0f} tok/s "
        f"({100 * res['frac_hbm']:.1f}% of HBM peak)")
    # the host-pointer drop-in (synchronous, x and out in host memory), the
    # entry point bound once so the loop measures the call, not Python
    x = synth.normal(9, synth.S_X, (1, d.hidden), 0.0, 1.0)
    o = np.empty_like(x)
    fn = gdn.lib().omh_gdn_decode
    xp, op = gdn._ptr(x), gdn._ptr(o)
    for _ in range(5):
        gdn.check(fn(lays[0].li, 1, xp, op))
    ts = []
    for i in range(200):
        li = lays[i % N_LAYERS].li
        t0 = time.perf_counter()
        rc = fn(li, 1, xp, op)
        ts.append(time.perf_counter() - t0)
        gdn.check(rc)
    res["host_call_us_median"] = 1e6 * statistics.median(ts)
    res["host_call_note"] = ("omh_gdn_decode(li, 1, x, out) with host x/out, layers in turn: x through pinned staging "
                             "and one async copy, the 3 launches, out written by out_proj into mapped pinned memory, "
                             "stream sync; wall clock per call from Python (ctypes), median of 200")
    log(f"host-pointer omh_gdn_decode(li, 1, ...): {res['host_call_us_median']:.1f} us per call")
    for L in lays:
        L.free()
    hip.device_synchronize()
    return res


def bench_prefill_block(hip, gdn, synth, T, steps, warmup):
    """Row f2 at prefill size: the whole GDN layer (int8 in_proj 2048 -> 12352
    with fp32 b/a rows, core, int8 out_proj 4096 -> 2048) over T tokens of
    one sequence, and the core alone on the same layer; the difference is
    the two projections (with their x-split launches)."""
    from overhang_amd.dims import Q35B
    d = Q35B
    w = quantized(synth.layer_weights(d, 6))
    L = gdn.GdnLayer(2200, d, w, max_seqs=1)
    x = hip.Buffer.from_numpy(synth.normal(10, synth.S_X, (T, d.hidden), 0.0, 1.0))
    out = hip.Buffer(T * d.hidden * 4)
    st = hip.Stream()
    el, _, _ = time_launches(hip, st, lambda k: gdn.prefill_dev(L.li, 0, T, x, out, stream=st), steps, warmup)
    t_layer = el / steps
    inp = synth.core_inputs(d, T, 11)
    dev = {k: hip.Buffer.from_numpy(v) for k, v in inp.items()}
    core = hip.Buffer(T * d.val_dim * 4)
    el2, _, _ = time_launches(hip, st, lambda k: gdn.prefill_core_dev(L.li, 0, T, dev["qkv"], dev["z"], dev["a"],
                                                                       dev["b"], core, stream=st), steps, warmup)
    t_core = el2 / steps
    L.free()
    t_proj = t_layer - t_core
    macs = T * (d.hidden * (d.conv_dim + d.val_dim + 2 * d.vh) + d.val_dim * d.hidden)
    tf = 2 * macs / t_proj / 1e12
    peak = INT8_MFMA_TOPS / 3
    res = {"T": T, "us_layer": 1e6 * t_layer, "us_core": 1e6 * t_core, "us_projections": 1e6 * t_proj,
           "tok_s_layer": T / t_layer, "proj_flops": 2 * macs, "proj_TFLOPs": tf,
           "roofline": {"bound": "mfma", "achieved": round(tf, 1), "peak": round(peak, 1), "unit": "TFLOP/s",
                        "frac": tf / peak,
                        "basis": "algorithmic int8 x fp32 multiply-adds of both projections x 2 per second; x "
                                 "enters the int8 matrix cores as three int8 planes, so each costs three int8 "
                                 "products and the bound is the dense int8 MFMA peak (5.0 POP/s) / 3"},
           "note": "35B GDN layer, int8 [qkv|z] in_proj + fp32 b/a rows, int8 out_proj; projections = "
                   "whole-layer prefill minus core-only prefill on the same layer"}
    log(f"prefill block T={T}: layer {1e6 * t_layer:.0f} us, core {1e6 * t_core:.0f} us, projections "
        f"{1e6 * t_proj:.0f} us = {tf:.0f} TFLOP/s")
    return res


def copy_probe(hip, nbytes, steps, warmup):
    """Device-to-device copy of nbytes (reads nbytes, writes nbytes): the HBM
    bandwidth a plain copy reaches on this box, next to the spec peak.  The
    buffers are far larger than the 256 MB Infinity Cache."""
    src, dst = hip.Buffer(nbytes), hip.Buffer(nbytes)
    st = hip.Stream()

    def one(k):
        hip.ok(hip.rt().hipMemcpyAsync(dst.ptr, src.ptr, nbytes, hip.D2D, st.cuda_stream))

    el, _, _ = time_launches(hip, st, one, steps, warmup)
    src.close()
    dst.close()
    t = el / steps
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": 1e6 * t, "GBs": 2 * nbytes / t / 1e9}


def prefill_flops(d, T, C=64):
    """Algorithmic FLOPs of the chunked WY/UT prefill of T tokens (per layer):
    per value head and chunk 2C^2(3kd + 2vd) for K K^T, Q K^T, W, U and
    Aqk v_new, 6 C kd vd for W S, (Q e^g) S and the state update, and C^3/3
    for the triangular inverse."""
    nc = -(-T // C)
    return d.vh * nc * (2 * C * C * (3 * d.kd + 2 * d.vd) + 6 * C * d.kd * d.vd + C ** 3 / 3)


def prefill_bytes(d, T):
    """Compulsory HBM bytes of a core prefill of T tokens: q, k (read as
    mixed_qkv), v, z in; core out; a, b in; the state read and written."""
    return (2 * T * d.kh * d.kd * 4 + 2 * T * d.vh * d.vd * 4 + 2 * T * d.vh * 4
            + 2 * d.state_bytes)


def bench_prefill(hip, gdn, synth, T, steps, warmup):
    from overhang_amd.dims import Q35B
    d = Q35B
    w = synth.layer_weights(d, 0, projections=False)
    L = gdn.GdnLayer(2000, d, w, max_seqs=1)
    inp = synth.core_inputs(d, T, 7)
    dev = {k: hip.Buffer.from_numpy(v) for k, v in inp.items()}
    core = hip.Buffer(T * d.val_dim * 4)
    st = hip.Stream()

    def one(k):
        gdn.prefill_core_dev(L.li, 0, T, dev["qkv"], dev["z"], dev["a"], dev["b"], core, stream=st)

    el, durs, _ = time_launches(hip, st, one, steps, warmup)
    L.free()
    t = el / steps
    fl = prefill_flops(d, T)
    by = prefill_bytes(d, T)
    tf = fl / t / 1e12
    peak = FP32_MFMA_TFLOPS
    # attainable roofline at this arithmetic intensity
    attain = min(peak, fl / by * HBM_PEAK_GBS / 1e3)
    out = {"T": T, "chunk": 64, "math": "fp32", "tok_s": T * steps / el, "us_per_call": 1e6 * t,
           "flops_per_call": fl, "TFLOPs": tf, "peak_TFLOPs": round(peak, 1),
           "frac_fp32_mfma": tf / FP32_MFMA_TFLOPS, "frac_peak": tf / peak, "frac_attainable": tf / attain,
           "hbm_bytes_alg": by, "recurrent_equiv_GFLOP": 7 * d.vh * T * d.kd * d.vd / 1e9,
           "note": "one GDN layer core (3 launches: WY/chunk (conv, norms, gates, triangular solve, "
                   "panels), scan, gated norm with the conv-history commit), "
                   "kh=16 vh=32 kd=vd=128, fp32 I/O, state carried across calls, fp32 MFMA"}
    log(f"prefill T={T}: {1e6 * t:.0f} us/layer, {out['tok_s']:.3g} tok/s, {tf:.1f} TFLOP/s "
        f"({100 * out['frac_peak']:.1f}% of the {peak:.0f} TFLOP/s matrix-core bound)")
    return out


def bench_prefill_warm(hip, gdn, synth, T, warm, steps, warmup):
    """Config 4: T-token prefill calls continuing from the state left by a
    warm-up prefill of `warm` tokens, gate logits a ~ N(-2, 1).  Inputs are a
    seeded 4096-token block repeated (generating T fresh 35B-width rows on the
    host would dominate the run); every call does the same work."""
    from overhang_amd.dims import Q35B
    d = Q35B
    w = synth.layer_weights(d, 1, projections=False)
    L = gdn.GdnLayer(2001, d, w, max_seqs=1)
    blk = synth.core_inputs(d, 4096, 11, a_mean=-2.0)
    rep = -(-max(T, warm) // 4096)
    dev = {k: hip.Buffer.from_numpy(np.tile(v, (rep, 1))) for k, v in blk.items()}
    core = hip.Buffer(max(T, warm) * d.val_dim * 4)
    st = hip.Stream()
    gdn.prefill_core_dev(L.li, 0, warm, dev["qkv"], dev["z"], dev["a"], dev["b"], core, stream=st)

    def one(k):
        gdn.prefill_core_dev(L.li, 0, T, dev["qkv"], dev["z"], dev["a"], dev["b"], core, stream=st)

    el, durs, _ = time_launches(hip, st, one, steps, warmup)
    L.free()
    t = el / steps
    fl = prefill_flops(d, T)
    tf = fl / t / 1e12
    out = {"T": T, "warm_tokens": warm, "chunk": 64, "tok_s": T * steps / el, "us_per_call": 1e6 * t,
           "flops_per_call": fl, "TFLOPs": tf, "frac_fp32_mfma": tf / FP32_MFMA_TFLOPS,
           "hbm_bytes_alg": prefill_bytes(d, T),
           "note": "config 4: one GDN layer core, T-token prefill continuing from the state of a "
                   f"{warm}-token prefill, a ~ N(-2,1), 35B head shape, fp32"}
    log(f"prefill warm-append T={T}: {1e6 * t:.0f} us/call, {out['tok_s']:.3g} tok/s, {tf:.1f} TFLOP/s "
        f"({100 * out['frac_fp32_mfma']:.1f}% of fp32 MFMA peak)")
    return out


def block_bytes(d, B):
    """Compulsory HBM bytes of one batched decode step of the whole GDN block
    with int8 projections: in_proj weights ([qkv|z] int8 + per-row scales,
    [b|a] fp32), out_proj int8 + scales, each sequence's recurrent and conv
    state read and written, x in and out."""
    n_q = d.conv_dim + d.val_dim
    w_in = n_q * d.hidden + 4 * n_q + 2 * d.vh * d.hidden * 4
    w_out = d.hidden * d.val_dim + 4 * d.hidden
    state = 2 * (d.state_bytes + 4 * d.conv_dim * (d.K - 1))
    return w_in + w_out + B * state + 2 * B * d.hidden * 4


def bench_block(hip, gdn, synth, B, steps, warmup):
    """Config 5: one decode step of the whole GDN block (int8 in_proj -> conv ->
    recurrence -> gated norm -> int8 out_proj) for B independent sequences,
    each with its own state, rotating over >1 GiB of layer states."""
    from overhang_amd.dims import Q35B
    d = Q35B
    w = synth.layer_weights(d, 5)
    per = B * (d.state_bytes + 4 * d.conv_dim * (d.K - 1))
    nrot = max(2, math.ceil(ROTATE_BYTES / per))
    lays = [gdn.GdnLayer(3000 + i, d, w, max_seqs=B, int8=True) for i in range(nrot)]
    x = hip.Buffer.from_numpy(synth.normal(7, synth.S_X, (B, d.hidden), 0.0, 1.0))
    out = hip.Buffer(B * d.hidden * 4)
    st = hip.Stream()

    def one(k):
        gdn.decode_dev(lays[k % nrot].li, B, x, out, stream=st)

    el, durs, _ = time_launches(hip, st, one, steps, warmup)
    t = el / steps
    by = block_bytes(d, B)
    gbs = by / t / 1e9
    # the same steps captured in HIP graphs (two steps of one layer per graph,
    # one graph per rotated layer) and replayed, as a serving loop issues them
    graphs = [hip.Graph(st, lambda L=L: [gdn.decode_dev(L.li, B, x, out, stream=st),
                                          gdn.decode_dev(L.li, B, x, out, stream=st)]) for L in lays]
    n = max(steps // 2, 5)
    el_g, _, _ = time_launches(hip, st, lambda k: graphs[k % nrot].launch(), n, warmup)
    for gr in graphs:
        gr.close()
    for L in lays:
        L.free()
    t_g = el_g / (2 * n)
    gbs_g = by / t_g / 1e9
    res = {"B": B, "us_per_step": 1e6 * t, "tok_s": B / t, "alg_bytes": by, "achieved_GBs": gbs,
           "frac_hbm": gbs / HBM_PEAK_GBS,
           "graph_us_per_step": 1e6 * t_g, "graph_achieved_GBs": gbs_g, "graph_frac_hbm": gbs_g / HBM_PEAK_GBS,
           "note": "config 5: whole GDN block, one token for each of B sequences, int8 [qkv|z] in_proj and "
                   "out_proj dequantised in-kernel, fp32 b/a rows, 35B shape; tok_s is per layer; us_per_step "
                   "from back-to-back stream launches, graph_us_per_step from HIP graph replays of the same steps"}
    log(f"block B={B}: {1e6 * t:.1f} us/step, {gbs:.0f} GB/s ({100 * res['frac_hbm']:.1f}% of HBM peak); "
        f"graph replay {1e6 * t_g:.1f} us/step ({100 * res['graph_frac_hbm']:.1f}%)")
    return res


ATTN_SHAPE = (2048, 16, 2, 256, 64)         # hidden, query heads, kv heads, head_dim, rot_dim (35B-A3B)


def attn_bytes(n, int8=True):
    """Compulsory HBM bytes of one decode token of the gated attention layer
    at n visible positions: the q/k/v and o projection weights (int8 + per-row
    scales), the K and V cache rows read, x in and out."""
    D, H, KV, hd, _ = ATTN_SHAPE
    rows = 2 * H * hd + 2 * KV * hd
    eb = 1 if int8 else 4
    w = (rows * D + D * H * hd) * eb + (4 * (rows + D) if int8 else 0)
    return w + 2 * KV * n * hd * 4 + 2 * D * 4


def bench_attn(hip, gdn, n, steps, warmup, nseq=8):
    """One decode token of the gated full-attention layer (engines/qwen.c:366-425)
    at the 35B-A3B attention shape with int8 projections, at position n - 1
    (n visible keys), rotating over nseq sequences' caches (> 1 GiB at
    n = 32768) so no step finds its cache in the last-level cache.  The
    caches hold zeros outside the rows the steps write; the kernels' work
    does not depend on the values."""
    D, H, KV, hd, rot = ATTN_SHAPE
    rng = np.random.default_rng(9)
    w = {"W_q": rng.normal(0, 0.02, (2 * H * hd, D)).astype(np.float32),
         "W_k": rng.normal(0, 0.02, (KV * hd, D)).astype(np.float32),
         "W_v": rng.normal(0, 0.02, (KV * hd, D)).astype(np.float32),
         "W_o": rng.normal(0, 0.02, (D, H * hd)).astype(np.float32),
         "q_norm": rng.normal(0, 0.1, hd).astype(np.float32),
         "k_norm": rng.normal(0, 0.1, hd).astype(np.float32)}
    L = gdn.AttnLayer(4000, D, H, KV, hd, rot, 1e7, 1e-6, n, w, max_seqs=nseq, int8=True)
    x = hip.Buffer.from_numpy(rng.normal(0, 1, (1, D)).astype(np.float32))
    out = hip.Buffer(D * 4)
    st = hip.Stream()

    def one(k):
        gdn.attn_forward_dev(L.li, k % nseq, n - 1, 1, x, out, stream=st)

    el, durs, _ = time_launches(hip, st, one, steps, warmup)
    L.free()
    t = el / steps
    by = attn_bytes(n)
    gbs = by / t / 1e9
    res = {"n": n, "us_per_step": 1e6 * t, "tok_s": 1 / t, "alg_bytes": by, "achieved_GBs": gbs,
           "frac_hbm": gbs / HBM_PEAK_GBS,
           "note": "gated full-attention layer, one decode token at n visible positions, hidden 2048, "
                   "16 query / 2 kv heads of 256, int8 q/k/v/o projections; 5 launches per token"}
    log(f"attn n={n}: {1e6 * t:.1f} us/step, {gbs:.0f} GB/s ({100 * res['frac_hbm']:.1f}% of HBM peak)")
    return res


def attn_prefill_flops(T, pos=0):
    """Algorithmic flops of the causal attention core for T new tokens at
    positions pos .. pos+T-1 (35B-A3B attention shape): per query head and
    token t, 2 hd flops per visible key for q.k and 2 hd for p.v."""
    D, H, KV, hd, rot = ATTN_SHAPE
    keys = T * pos + T * (T + 1) / 2
    return 4.0 * H * hd * keys


def bench_attn_prefill(hip, gdn, T, steps, warmup):
    """One prompt step of the gated full-attention layer at the 35B-A3B
    attention shape: T tokens of one sequence at positions 0 .. T-1 through
    omh_attn_forward_dev (int8 q/k/v/o projections, norm + RoPE + cache
    write, causal attention, gate)."""
    D, H, KV, hd, rot = ATTN_SHAPE
    rng = np.random.default_rng(19)
    w = {"W_q": rng.normal(0, 0.02, (2 * H * hd, D)).astype(np.float32),
         "W_k": rng.normal(0, 0.02, (KV * hd, D)).astype(np.float32),
         "W_v": rng.normal(0, 0.02, (KV * hd, D)).astype(np.float32),
         "W_o": rng.normal(0, 0.02, (D, H * hd)).astype(np.float32),
         "q_norm": rng.normal(0, 0.1, hd).astype(np.float32),
         "k_norm": rng.normal(0, 0.1, hd).astype(np.float32)}
    L = gdn.AttnLayer(4010, D, H, KV, hd, rot, 1e7, 1e-6, T, w, max_seqs=1, int8=True)
    x = hip.Buffer.from_numpy(rng.normal(0, 1, (T, D)).astype(np.float32))
    out = hip.Buffer(T * D * 4)
    st = hip.Stream()

    def one(k):
        gdn.attn_forward_dev(L.li, 0, 0, T, x, out, stream=st)

    el, _, _ = time_launches(hip, st, one, steps, warmup)
    L.free()
    t = el / steps
    fl = attn_prefill_flops(T)
    res = {"T": T, "us_per_call": 1e6 * t, "tok_s": T / t, "attn_flops": fl, "attn_TFLOPs_layer_time": fl / t / 1e12,
           "note": "gated full-attention layer prompt step, T tokens from position 0, hidden 2048, 16 query / 2 kv "
                   "heads of 256 (rot 64), int8 q/k/v/o projections; TFLOP/s = causal attention flops over the "
                   "whole layer's time"}
    log(f"attn prefill T={T}: {1e6 * t:.0f} us/call, {T / t:.3g} tok/s, attention {fl / t / 1e12:.1f} TFLOP/s "
        f"over the layer time")
    return res


def bench_snapshot(hip, gdn, synth, steps, warmup):
    """Speculative-decoding snapshot of one sequence's GDN state across the
    30 GDN layers of the 35B shape copied device to device into a spare
    sequence slot, one omh_gdn_state_copy_dev call (one launch), rotating
    over 4 groups of 30 layers so no step finds its state in the
    last-level cache."""
    from overhang_amd.dims import Q35B
    d = Q35B
    w = synth.layer_weights(d, 0, projections=False)
    R = 4                                  # layer groups rotated: 536 MB, beyond the last-level cache
    lays = [gdn.GdnLayer(3500 + i, d, w, max_seqs=2) for i in range(R * N_LAYERS)]
    st = hip.Stream()
    groups = [[L.li for L in lays[r * N_LAYERS:(r + 1) * N_LAYERS]] for r in range(R)]

    def one(k):
        gdn.state_copy_dev(groups[k % R], 0, 1, stream=st)

    el, _, _ = time_launches(hip, st, one, steps, warmup)
    for L in lays:
        L.free()
    t = el / steps
    per_layer = d.state_bytes + 4 * d.conv_dim * 4 + 4              # S, the conv ring, the phase
    by = 2 * N_LAYERS * per_layer                                   # read + write
    gbs = by / t / 1e9
    res = {"us_per_snapshot": 1e6 * t, "bytes": by, "achieved_GBs": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
           "note": "one sequence's state across 30 GDN layers (35B shape) copied device to device into a "
                   "spare slot: the snapshot (or rollback) of a speculative-decoding step"}
    log(f"state snapshot x {N_LAYERS} layers: {1e6 * t:.1f} us, {gbs:.0f} GB/s")
    return res


def cpu_prefill_baseline(synth, T=256, budget_s=8.0):
    """The oracle prefills token by token (the reference has no chunked CPU
    path): one layer core at the 35B shape over a bounded sample of T tokens."""
    import oracle
    from overhang_amd.dims import Q35B
    d = Q35B
    w = synth.layer_weights(d, 0, projections=False)
    inp = synth.core_inputs(d, T, 7)
    conv0 = np.zeros((d.conv_dim, d.K - 1), np.float32)
    S0 = np.zeros((d.vh, d.kd, d.vd), np.float32)
    oracle.core_seq(d, w, inp["qkv"][:8], inp["z"][:8], inp["a"][:8], inp["b"][:8], conv0, S0)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": T / med, "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{len(times)} runs of {T} tokens through one GDN layer core at the 35B shape, "
                      f"token by token (median {1e3 * med:.0f} ms per run)"}


def cpu_decode_baseline(synth, budget_s=10.0):
    """The oracle (reference GDN restated in C, OpenMP) on the host: one token
    through the GDN core of 30 layers at the 35B shape, each layer its own state."""
    import oracle
    from overhang_amd.dims import Q35B
    d = Q35B
    w = synth.layer_weights(d, 0, projections=False)
    conv0, S0 = synth.states(d, 0)
    inp = synth.core_inputs(d, N_LAYERS, 1)
    convs = [conv0.copy() for _ in range(N_LAYERS)]
    Ss = [S0.copy() for _ in range(N_LAYERS)]
    lib = oracle.lib()
    dd = oracle._dims(d)
    import ctypes as C
    core = np.empty(d.val_dim, np.float32)
    args = [oracle._c(w[k]) for k in ("conv_w", "A_log", "dt_bias", "gnorm")]

    def one_token():
        for l in range(N_LAYERS):
            lib.gdno_core_seq(C.byref(dd), *args, 1, inp["qkv"][l], inp["z"][l], inp["a"][l],
                              inp["b"][l], convs[l], Ss[l], core)

    one_token()                                  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        one_token()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": 1.0 / med, "unit": "tok/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"{len(times)} tokens x {N_LAYERS} layers of the GDN core at the 35B shape, B=1 "
                      f"(median per token {1e3 * med:.1f} ms)",
            "cpu_model": cpu_model()}


def cpu_model() -> str:
    """lscpu's model name, sockets x cores, and the threads this process may use."""
    import subprocess
    model, info = "unknown", {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                info[k.strip()] = v.strip()
        model = info.get("Model name", model)
    except (OSError, subprocess.SubprocessError):
        pass
    return (f"{model}; {info.get('Socket(s)', '?')} socket(s) x {info.get('Core(s) per socket', '?')} cores, "
            f"{info.get('CPU(s)', '?')} CPUs; nproc {len(os.sched_getaffinity(0))}")


def cpu_reference_layer(synth, budget_s=10.0):
    """The reference's own deltanet_step (engines/qwen.c:301-364, compiled
    from the reference sources into oracle/_ref with the reference's flags)
    on the whole GDN layer at the 35B shape with int8 projections, one token
    per call as the engine runs it; tok/s for 30 such layers."""
    import oracle
    from overhang_amd.dims import Q35B
    if oracle.ref_lib() is None:
        return None
    d = Q35B
    R = oracle.RefLayer(d, synth.layer_weights(d, 5), int8=True)
    x = synth.normal(9, synth.S_X, (1, d.hidden), 0.0, 1.0)
    R.steps(x)
    ts = []
    t_start = time.perf_counter()
    while len(ts) < 5 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        R.steps(x)
        ts.append(time.perf_counter() - t0)
    R.close()
    med = statistics.median(ts)
    return {"value": 1.0 / (N_LAYERS * med), "unit": "tok/s", "cores": oracle.threads(), "kind": "reference",
            "ms_per_layer": 1e3 * med,
            "sample": f"{len(ts)} tokens through one whole GDN layer (int8 in/out projections, 35B shape) "
                      f"with the reference deltanet_step; tok/s = 1 / (30 x median per-layer time)",
            "cpu_model": cpu_model()}


def committed_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by a copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return rec


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--part", choices=("all", "decode", "headline", "prefill", "block", "attn", "attnp", "engine",
                                       "proj"),
                    default="all",
                    help="decode: the headline and its weights-rotated form; headline: the headline launch "
                         "alone (for profiling); prefill: the T=4096 and T=32768 "
                         "prefills only; block: the config 5 int8 block at B=64 only; attn: the gated "
                         "attention layer's decode token at 32768 positions only; engine: the 30-layer "
                         "whole-block B=1 chain in a HIP graph; proj: the T=4096 int8 layer prefill; attnp: the "
                         "attention layer's T=4096 prompt step")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the GDN layer needs no collectives and this build "
              "runs single-GPU only (--gpus 1).", file=sys.stderr)
        sys.exit(2)
    from overhang_amd import gdn, hip, synth
    gdn.require_gpu()
    log("device: gfx950 ready")
    if a.part == "prefill":
        pre = bench_prefill(hip, gdn, synth, 4096, max(a.steps // 5, 3), a.warmup)
        warm = bench_prefill_warm(hip, gdn, synth, 32768, 8192, 3, 1)
        print(json.dumps({"prefill": pre, "prefill_T32768_warm": warm}), flush=True)
        return
    if a.part == "attn":
        print(json.dumps({"attn_decode_n32768": bench_attn(hip, gdn, 32768, max(a.steps // 2, 10), a.warmup)}),
              flush=True)
        return
    if a.part == "attnp":
        print(json.dumps({"attn_prefill_T4096": bench_attn_prefill(hip, gdn, 4096, max(a.steps // 10, 3), 1)}),
              flush=True)
        return
    if a.part == "engine":
        print(json.dumps({"engine_block_B1": bench_engine_block(hip, gdn, synth, a.steps, a.warmup)}), flush=True)
        return
    if a.part == "proj":
        print(json.dumps({"prefill_block_int8_T4096": bench_prefill_block(hip, gdn, synth, 4096, max(a.steps // 5, 3),
                                                                          a.warmup)}), flush=True)
        return
    if a.part == "block":
        print(json.dumps({"block_int8_B64": bench_block(hip, gdn, synth, 64, max(a.steps // 2, 10), a.warmup)}),
              flush=True)
        return
    fused, engine, sweep, alg_bytes, R = bench_decode(hip, gdn, synth, a.steps, a.warmup,
                                                      full=a.part == "all", rotated=a.part != "headline")
    pre = warm = block = attn = attnp = snap = eng = preb = None
    if a.part == "all":
        eng = bench_engine_block(hip, gdn, synth, a.steps, a.warmup)
        preb = bench_prefill_block(hip, gdn, synth, 4096, max(a.steps // 5, 5), a.warmup)
        attn = bench_attn(hip, gdn, 32768, max(a.steps // 2, 10), a.warmup)
        attnp = bench_attn_prefill(hip, gdn, 4096, 5, 1)
        snap = bench_snapshot(hip, gdn, synth, max(a.steps // 2, 10), a.warmup)
        pre = bench_prefill(hip, gdn, synth, 4096, max(a.steps // 5, 5), a.warmup)
        warm = bench_prefill_warm(hip, gdn, synth, 32768, 8192, 5, 1)
        block = bench_block(hip, gdn, synth, 64, max(a.steps // 2, 10), a.warmup)
    probe = copy_probe(hip, 1 << 29, 20, 3)
    log(f"copy probe: {probe['GBs']:.0f} GB/s (D2D copy of 512 MiB)")
    cpu = None
    if not a.no_cpu:
        log("cpu baseline (oracle, OpenMP) ...")
        cpu = cpu_decode_baseline(synth)
        log(f"cpu baseline: {cpu['value']:.1f} tok/s on {cpu['cores']} threads")
        cpu_ref = cpu_reference_layer(synth)
        if cpu_ref is not None:
            log(f"cpu reference deltanet_step (whole layer, int8): {cpu_ref['ms_per_layer']:.1f} ms per layer")
            if eng is not None:
                eng["cpu_baseline"] = cpu_ref
        if pre is not None:
            pre["cpu_baseline"] = cpu_prefill_baseline(synth)
            log(f"cpu prefill baseline: {pre['cpu_baseline']['value']:.1f} tok/s")
    ach = fused["achieved_GBs"]
    kname = "gdn_decode_paired_kernel<128, 128, 2>"
    tr = committed_traffic(kname)
    line = {
        "metric": METRIC,
        "value": round(fused["tok_s"], 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(fused["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (splitmix64/Box-Muller, seeded); random-init GDN weights of the 35B GDN shape",
        "config": {"workload": "GDN core decode, 1 token x 30 layers (one launch), B=1 (one of R sequence slots "
                               "per step, rotating), "
                               "kh=16 vh=32 kd=vd=128, fp32 state, pre-projected inputs",
                   "layers": N_LAYERS, "batch": 1,
                   "state_rotation_GiB": round(R * N_LAYERS * 2.19e6 / 2**30, 2)},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": None if tr is None else tr["bytes_per_launch"],
                     "kernel": kname, "kernel_us": round(fused["kernel_us"], 2),
                     "alg_bytes_per_launch": alg_bytes,
                     "traffic_source": None if tr is None else tr["source"],
                     # the headline basis is the recurrent state alone; the step's full
                     # compulsory bytes per layer (conv state read + write, conv weights,
                     # inputs and output) are 4.59 MB against the state's 4.19 MB
                     "full_compulsory_bytes_per_launch": N_LAYERS * FULL_COMPULSORY_PER_LAYER,
                     "frac_full_compulsory": round(N_LAYERS * FULL_COMPULSORY_PER_LAYER / (fused["kernel_us"] * 1e-6)
                                                   / 1e9 / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
        "hbm_copy_probe": probe,
        "prefill_T4096": pre,
        "prefill_T32768_warm": warm,
        "block_int8_B64": block,
        "attn_decode_n32768": attn,
        "attn_prefill_T4096": attnp,
        "gdn_state_snapshot_30layers": snap,
        "decode_engine_order": engine,
        "decode_weights_rotated": fused.get("weights_rotated"),
        "engine_block_B1": eng,
        "prefill_block_int8_T4096": preb,
        "decode_batch_sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
