#!/usr/bin/env python3
"""GDN layer throughput on one MI355X, next to the CPU reference GDN.

Headline (the JSON line's `value`): decode of one token through the GDN core
of 30 layers at the Qwen3.6-35B-A3B GDN shape (kh=16, vh=32, kd=vd=128),
batch 1, pre-projected inputs (mixed_qkv, z, a, b), fp32 state.  The 30
layers' inputs are independent, so one launch serves all 30; every step uses
a different set of 30 layer states out of >1 GiB so the 256 MB Infinity
Cache cannot hold them (each step reads and writes 126 MB of state from HBM).

Also reported: the same step launched layer by layer (the order an engine
runs it), a batch sweep B=1..64 of one-layer launches, and the CPU oracle
(the reference GDN restated in C, OpenMP) on the host cores.

usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
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
BF16_MFMA_TFLOPS = 2500.0
N_LAYERS = 30
ROTATE_BYTES = 1 << 30


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


def bench_decode(hip, gdn, synth, steps, warmup):
    from overhang_amd.dims import Q35B
    d = Q35B
    per_layer = d.state_bytes + 4 * d.conv_dim * (d.K - 1)
    R = math.ceil(ROTATE_BYTES / (N_LAYERS * per_layer))
    log(f"decode: {R} x {N_LAYERS} layers, {R * N_LAYERS * per_layer / 2**30:.2f} GiB of state")
    w = synth.layer_weights(d, 0, projections=False)
    conv0, S0 = synth.states(d, 0)
    lays = make_layers(gdn, d, 0, R * N_LAYERS, 1, w, conv0, S0)
    inp = synth.core_inputs(d, N_LAYERS, 1)                # [30][...] = [nl][B=1][...]
    dev = {k: hip.Buffer.from_numpy(v) for k, v in inp.items()}
    row = {k: v.shape[1] * 4 for k, v in inp.items()}
    core = hip.Buffer(N_LAYERS * d.val_dim * 4)
    st = hip.Stream()
    groups = [[lays[r * N_LAYERS + l].li for l in range(N_LAYERS)] for r in range(R)]

    def step_fused(k):
        gdn.decode_core_dev(groups[k % R], 1, dev["qkv"], dev["z"], dev["a"], dev["b"], core, stream=st)

    el, durs, wall = time_launches(hip, st, step_fused, steps, warmup)
    alg_bytes = N_LAYERS * 2 * d.state_bytes                # state read + write, 30 layers
    kern = statistics.mean(durs)
    fused = {"tok_s": steps / el, "ms_per_step": 1e3 * el / steps, "kernel_us": 1e6 * kern,
             "achieved_GBs": alg_bytes / kern / 1e9, "wall_s": wall}
    log(f"decode fused 30-layer launch: {fused['tok_s']:.0f} tok/s, kernel {fused['kernel_us']:.1f} us, "
        f"{fused['achieved_GBs']:.0f} GB/s")

    # engine order: one launch per layer
    def step_layers(k):
        g = groups[k % R]
        for l in range(N_LAYERS):
            gdn.decode_core_dev([g[l]], 1, *(dev[nm].at(l * row[nm]) for nm in ("qkv", "z", "a", "b")),
                                core.at(l * d.val_dim * 4), stream=st)

    el2, durs2, _ = time_launches(hip, st, step_layers, max(steps // 2, 5), warmup)
    n2 = max(steps // 2, 5)
    k2 = statistics.mean(durs2) / N_LAYERS
    engine = {"tok_s": n2 / el2, "ms_per_step": 1e3 * el2 / n2, "kernel_us_per_layer_incl_gaps": 1e6 * k2,
              "note": "30 dependent one-layer launches per token, as an engine issues them"}
    log(f"decode engine order (30 launches/token): {engine['tok_s']:.0f} tok/s")
    for L in lays:
        L.free()
    hip.device_synchronize()

    # batch sweep: one layer per launch, B sequences, rotating over >1 GiB
    sweep = []
    Bmax = 64
    nrot = max(2, math.ceil(ROTATE_BYTES / (Bmax * per_layer)))
    lays = make_layers(gdn, d, 1000, nrot, Bmax, w, conv0, S0)
    inpB = synth.core_inputs(d, 1, 2, B=Bmax)
    devB = {k: hip.Buffer.from_numpy(np.ascontiguousarray(v[:, 0])) for k, v in inpB.items()}
    coreB = hip.Buffer(Bmax * d.val_dim * 4)
    for B in (1, 2, 4, 8, 16, 32, 64):
        def stepB(k, B=B):
            gdn.decode_core_dev([lays[k % nrot].li], B, devB["qkv"], devB["z"], devB["a"], devB["b"], coreB,
                                stream=st)
        nsteps = max(steps, 20)
        elB, dB, _ = time_launches(hip, st, stepB, nsteps, warmup)
        kb = statistics.mean(dB)
        gbs = B * 2 * d.state_bytes / kb / 1e9
        sweep.append({"B": B, "kernel_us": 1e6 * kb, "achieved_GBs": gbs, "frac_hbm": gbs / HBM_PEAK_GBS,
                      "tok_s_30_layers": B / (N_LAYERS * kb)})
        log(f"decode sweep B={B}: kernel {1e6 * kb:.1f} us, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}%)")
    for L in lays:
        L.free()
    hip.device_synchronize()
    return fused, engine, sweep, alg_bytes, R


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
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the GDN layer needs no collectives and this build "
              "runs single-GPU only (--gpus 1).", file=sys.stderr)
        sys.exit(2)
    from overhang_amd import gdn, hip, synth
    gdn.require_gpu()
    log("device: gfx950 ready")
    fused, engine, sweep, alg_bytes, R = bench_decode(hip, gdn, synth, a.steps, a.warmup)
    cpu = None
    if not a.no_cpu:
        log("cpu baseline (oracle, OpenMP) ...")
        cpu = cpu_decode_baseline(synth)
        log(f"cpu baseline: {cpu['value']:.1f} tok/s on {cpu['cores']} threads")
    ach = fused["achieved_GBs"]
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
        "config": {"workload": "GDN core decode, 1 token x 30 layers (one launch), B=1, "
                               "kh=16 vh=32 kd=vd=128, fp32 state, pre-projected inputs",
                   "layers": N_LAYERS, "batch": 1, "state_rotation_GiB": round(R * N_LAYERS * 2.19e6 / 2**30, 2)},
        "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gdn_decode_core_kernel<128,128,2>", "kernel_us": round(fused["kernel_us"], 2),
                     "alg_bytes_per_launch": alg_bytes},
        "cpu_baseline": cpu,
        "decode_engine_order": engine,
        "decode_batch_sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
