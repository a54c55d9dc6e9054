"""GPU parity of the decode path (one token per call) through the C-ABI.

Against the reference's golden vectors (tests/golden, written by the
reference deltanet_step) and the CPU oracle on seeded inputs, at the
tolerance in tests/tol.py.  Every call goes through libom_hip.so."""
import numpy as np
import pytest

import oracle
from overhang_amd import gdn, synth
from overhang_amd.dims import GdnDims, Q35B, CFG1
from tests import fixtures
from tests.tol import assert_close

pytestmark = pytest.mark.gpu

_next_li = [100]


def new_li():
    _next_li[0] += 1
    return _next_li[0]


# every decode kernel: chosen by launch size, paired heads, one slice per head
VARIANTS = [{}, {"OMH_DECODE_KERNEL": "paired"}, {"OMH_DECODE_KERNEL": "sliced", "OMH_DECODE_NCS": "1"}]
VARIANT_IDS = ["auto", "paired", "sliced1"]


@pytest.fixture(params=VARIANTS, ids=VARIANT_IDS)
def variant(request, monkeypatch):
    for k in ("OMH_DECODE_KERNEL", "OMH_DECODE_NCS"):
        monkeypatch.delenv(k, raising=False)
    for k, v in request.param.items():
        monkeypatch.setenv(k, v)
    return request.param


@pytest.mark.parametrize("name", fixtures.CORE_FIXTURES)
def test_decode_core_matches_reference_golden(name, variant):
    d, w, inp, (conv, S), exp = fixtures.load(name)
    L = gdn.GdnLayer(new_li(), d, w)
    L.set_state(0, conv, S)
    T = inp["qkv"].shape[0]
    core = np.stack([L.decode_core(inp["qkv"][t:t + 1], inp["z"][t:t + 1], inp["a"][t:t + 1],
                                   inp["b"][t:t + 1])[0] for t in range(T)])
    conv2, S2 = L.get_state(0)
    assert_close(core, exp["core"], what=f"{name} core")
    assert_close(S2, exp["S"], what=f"{name} S")
    assert np.array_equal(conv2, exp["conv"]), "conv history is a copy of inputs: must be exact"
    L.free()


@pytest.mark.parametrize("name", fixtures.LAYER_FIXTURES)
def test_decode_layer_matches_reference_golden(name, variant):
    d, w, inp, (conv, S), exp = fixtures.load(name)
    L = gdn.GdnLayer(new_li(), d, w, int8=exp["int8"])
    L.set_state(0, conv, S)
    x = inp["x"]
    out = np.concatenate([L.decode(x[t:t + 1]) for t in range(x.shape[0])])
    conv2, S2 = L.get_state(0)
    assert_close(out, exp["out"], what=f"{name} out")
    assert_close(S2, exp["S"], what=f"{name} S")
    assert_close(conv2, exp["conv"], atol=1e-5, rtol=1e-5, what=f"{name} conv")
    L.free()


def test_decode_core_35b_shape_batched_vs_oracle(variant):
    """Qwen3.6-35B-A3B GDN shape, 3 sequences with distinct states, 4 tokens."""
    d = Q35B
    w = synth.layer_weights(d, 31, gnorm_std=0.1, projections=False)
    B, T = 3, 4
    inp = synth.core_inputs(d, T, 31, B=B)
    conv0, S0 = synth.states(d, 31, B=B)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=B)
    for s in range(B):
        L.set_state(s, conv0[s], S0[s])
    got = np.stack([L.decode_core(inp["qkv"][:, t], inp["z"][:, t], inp["a"][:, t], inp["b"][:, t])
                    for t in range(T)], axis=1)
    for s in range(B):
        ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"][s], inp["z"][s], inp["a"][s], inp["b"][s],
                                          conv0[s], S0[s])
        conv, S = L.get_state(s)
        assert_close(got[s], ref, what=f"seq {s} core")
        assert_close(S, Sref, what=f"seq {s} S")
        assert np.array_equal(conv, cref)
    L.free()


def test_decode_core_35b_large_batches_run_as_chunks():
    """At the 35B shape a call with more than 32 sequences runs as several
    launches (each one round of resident workgroups), with the ring phases
    carried across them: batch sizes 48, 40, 48, 33 over four steps, every
    sequence checked against its own oracle run."""
    d = Q35B
    w = synth.layer_weights(d, 33, gnorm_std=0.1, projections=False)
    nmax = 48
    conv0, S0 = synth.states(d, 33, B=nmax)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=nmax)
    for s in range(nmax):
        L.set_state(s, conv0[s], S0[s])
    plan = [48, 40, 48, 33]
    inp = synth.core_inputs(d, len(plan), 34, B=nmax)
    fed = {s: [] for s in range(nmax)}
    outs = {s: [] for s in range(nmax)}
    for t, B in enumerate(plan):
        core = L.decode_core(inp["qkv"][:B, t], inp["z"][:B, t], inp["a"][:B, t], inp["b"][:B, t])
        for s in range(B):
            fed[s].append(t)
            outs[s].append(core[s])
    for s in (0, 23, 24, 32, 33, 39, 40, 47):
        ts = fed[s]
        ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"][s, ts], inp["z"][s, ts], inp["a"][s, ts],
                                          inp["b"][s, ts], conv0[s], S0[s])
        conv, S = L.get_state(s)
        assert_close(np.stack(outs[s]), ref, what=f"seq {s}")
        assert_close(S, Sref, what=f"seq {s} S")
        assert np.array_equal(conv, cref), f"seq {s} conv history"
    L.free()


def test_multi_layer_dev_call_equals_per_layer_calls(variant):
    from overhang_amd import hip
    d = CFG1
    nl, B = 5, 2
    lays, lays2 = [], []
    for l in range(nl):
        w = synth.layer_weights(d, 40 + l, gnorm_std=0.1, projections=False)
        conv0, S0 = synth.states(d, 40 + l, B=B)
        a = gdn.GdnLayer(new_li(), d, w, max_seqs=B)
        b = gdn.GdnLayer(new_li(), d, w, max_seqs=B)
        for s in range(B):
            a.set_state(s, conv0[s], S0[s])
            b.set_state(s, conv0[s], S0[s])
        lays.append(a)
        lays2.append(b)
    inp = synth.core_inputs(d, nl, 50, B=B)       # [B][nl][...] -> need [nl][B][...]
    host = {k: np.ascontiguousarray(np.swapaxes(v, 0, 1)) for k, v in inp.items()}
    dev = {k: hip.Buffer.from_numpy(v) for k, v in host.items()}
    core = hip.Buffer(nl * B * d.val_dim * 4)
    st = hip.Stream()
    gdn.decode_core_dev([L.li for L in lays], B, dev["qkv"], dev["z"], dev["a"], dev["b"], core, stream=st)
    st.synchronize()
    got = core.numpy((nl, B, d.val_dim))
    for l in range(nl):
        ref = lays2[l].decode_core(host["qkv"][l], host["z"][l], host["a"][l], host["b"][l])
        np.testing.assert_array_equal(got[l], ref)
        for s in range(B):
            c1, S1 = lays[l].get_state(s)
            c2, S2 = lays2[l].get_state(s)
            assert np.array_equal(c1, c2) and np.array_equal(S1, S2)
    for L in lays + lays2:
        L.free()


def test_state_roundtrip_reset_and_isolation():
    d = CFG1
    w = synth.layer_weights(d, 60, projections=False)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=3)
    conv0, S0 = synth.states(d, 60, B=3)
    for s in range(3):
        L.set_state(s, conv0[s], S0[s])
    for s in range(3):
        c, S = L.get_state(s)
        assert np.array_equal(c, conv0[s]) and np.array_equal(S, S0[s])
    L.reset(1)
    c, S = L.get_state(1)
    assert not c.any() and not S.any()
    c, S = L.get_state(2)
    assert np.array_equal(S, S0[2])
    # a B=1 call touches sequence 0 only
    inp = synth.core_inputs(d, 1, 61)
    L.decode_core(inp["qkv"], inp["z"], inp["a"], inp["b"])
    c, S = L.get_state(2)
    assert np.array_equal(S, S0[2]) and np.array_equal(c, conv0[2])
    L.reset(-1)
    for s in range(3):
        c, S = L.get_state(s)
        assert not c.any() and not S.any()
    L.free()


def test_argument_errors_are_reported():
    d = CFG1
    w = synth.layer_weights(d, 62, projections=False)
    with pytest.raises(gdn.OmhError) as e:
        gdn.GdnLayer(new_li(), GdnDims(2, 4, 48, 48, 4, 0), synth.layer_weights(GdnDims(2, 4, 48, 48, 4, 0), 0, projections=False))
    assert e.value.code == gdn.OMH_ERR_SHAPE
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=2)
    inp = synth.core_inputs(d, 3, 63)
    with pytest.raises(gdn.OmhError) as e:
        L.decode_core(inp["qkv"], inp["z"], inp["a"], inp["b"])      # B=3 > max_seqs
    assert e.value.code == gdn.OMH_ERR_ARG
    assert gdn.lib().omh_gdn_decode_core(4095, 1, None, None, None, None, None) == gdn.OMH_ERR_ARG
    with pytest.raises(gdn.OmhError):
        L.decode(np.zeros((1, 128), np.float32))                       # core-only layer
    L.free()


@pytest.mark.parametrize("K", [2, 3, 4])
@pytest.mark.parametrize("form", ["auto", "paired", "sliced1", "sliced4"])
def test_conv_widths_every_kernel(K, form, monkeypatch):
    """Conv widths 2-4 through every decode kernel, two sequences, seven
    steps each (the ring of four slots wraps), after a prefill of 5 tokens
    that leaves the ring at a phase other than 0: outputs, state and conv
    history against the oracle.  The sliced kernel requests every ring slot
    and picks the history slots by the phase afterwards; the paired kernel
    requests only the history slots."""
    for k in ("OMH_DECODE_KERNEL", "OMH_DECODE_NCS"):
        monkeypatch.delenv(k, raising=False)
    if form != "auto":
        monkeypatch.setenv("OMH_DECODE_KERNEL", "paired" if form == "paired" else "sliced")
        if form != "paired":
            monkeypatch.setenv("OMH_DECODE_NCS", form[-1])
    d = GdnDims(2, 4, 32, 32, K, 0)
    seed = 500 + 10 * K + len(form)
    w = synth.layer_weights(d, seed, gnorm_std=0.2, projections=False)
    conv0, S0 = synth.states(d, seed, B=2)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=2)
    for s_ in range(2):
        L.set_state(s_, conv0[s_], S0[s_])
    pre = synth.core_inputs(d, 5, seed + 1)
    L.prefill_core(0, pre["qkv"], pre["z"], pre["a"], pre["b"])
    _, c0, s0 = oracle.core_seq(d, w, pre["qkv"], pre["z"], pre["a"], pre["b"], conv0[0], S0[0])
    T = 7
    inp = synth.core_inputs(d, T, seed + 2, B=2)
    got = np.stack([L.decode_core(inp["qkv"][:, t], inp["z"][:, t], inp["a"][:, t], inp["b"][:, t])
                    for t in range(T)], axis=1)
    for s_, (cs, ss) in enumerate([(c0, s0), (conv0[1], S0[1])]):
        ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"][s_], inp["z"][s_], inp["a"][s_], inp["b"][s_], cs, ss)
        conv, S = L.get_state(s_)
        what = f"K={K} {form} seq{s_}"
        assert_close(got[s_], ref, what=what + " core")
        assert_close(S, Sref, what=what + " S")
        assert np.array_equal(conv, cref), what + ": conv history is a copy of the inputs"
    L.free()


@pytest.mark.parametrize("ncs", [1, 2, 4, 8])
def test_column_slices_agree_with_oracle(ncs, monkeypatch):
    """Every column-slice count (incl. the cross-slice gated-norm epilogue)."""
    monkeypatch.setenv("OMH_DECODE_KERNEL", "sliced")
    monkeypatch.setenv("OMH_DECODE_NCS", str(ncs))
    d = GdnDims(2, 4, 128, 128, 4, 0)
    w = synth.layer_weights(d, 70 + ncs, gnorm_std=0.2, projections=False)
    T = 3
    inp = synth.core_inputs(d, T, 70 + ncs)
    conv0, S0 = synth.states(d, 70 + ncs)
    L = gdn.GdnLayer(new_li(), d, w)
    L.set_state(0, conv0, S0)
    got = np.concatenate([L.decode_core(inp["qkv"][t:t + 1], inp["z"][t:t + 1], inp["a"][t:t + 1],
                                        inp["b"][t:t + 1]) for t in range(T)])
    ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"], conv0, S0)
    conv, S = L.get_state(0)
    assert_close(got, ref, what=f"ncs={ncs} core")
    assert_close(S, Sref, what=f"ncs={ncs} S")
    assert np.array_equal(conv, cref)
    L.free()


def test_varying_batch_keeps_each_sequence_history(variant):
    """Calls with B = 3, 1, 2, 3, 1 on one layer: sequences left out of a call
    keep their conv history and phase; each matches its own oracle run."""
    d = CFG1
    w = synth.layer_weights(d, 80, gnorm_std=0.1, projections=False)
    conv0, S0 = synth.states(d, 80, B=3)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=3)
    for s in range(3):
        L.set_state(s, conv0[s], S0[s])
    plan = [3, 1, 2, 3, 1, 3]
    inp = synth.core_inputs(d, len(plan), 81, B=3)
    fed = {s: [] for s in range(3)}
    outs = {s: [] for s in range(3)}
    for t, B in enumerate(plan):
        core = L.decode_core(inp["qkv"][:B, t], inp["z"][:B, t], inp["a"][:B, t], inp["b"][:B, t])
        for s in range(B):
            fed[s].append(t)
            outs[s].append(core[s])
    for s in range(3):
        ts = fed[s]
        ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"][s, ts], inp["z"][s, ts], inp["a"][s, ts],
                                          inp["b"][s, ts], conv0[s], S0[s])
        conv, S = L.get_state(s)
        assert_close(np.stack(outs[s]), ref, what=f"seq {s}")
        assert_close(S, Sref, what=f"seq {s} S")
        assert np.array_equal(conv, cref), f"seq {s} conv history"
    L.free()


def test_state_set_mid_stream_restarts_history(variant):
    """state_set after some decode steps (ring phase != 0) re-bases the ring."""
    d = CFG1
    w = synth.layer_weights(d, 90, projections=False)
    L = gdn.GdnLayer(new_li(), d, w)
    inp = synth.core_inputs(d, 7, 90)
    for t in range(5):
        L.decode_core(inp["qkv"][t:t + 1], inp["z"][t:t + 1], inp["a"][t:t + 1], inp["b"][t:t + 1])
    conv0, S0 = synth.states(d, 91)
    L.set_state(0, conv0, S0)
    c, S = L.get_state(0)
    assert np.array_equal(c, conv0) and np.array_equal(S, S0)
    got = np.concatenate([L.decode_core(inp["qkv"][t:t + 1], inp["z"][t:t + 1], inp["a"][t:t + 1],
                                        inp["b"][t:t + 1]) for t in (5, 6)])
    ref, cref, _ = oracle.core_seq(d, w, inp["qkv"][5:7], inp["z"][5:7], inp["a"][5:7], inp["b"][5:7],
                                   conv0, S0)
    assert_close(got, ref)
    assert np.array_equal(L.get_state(0)[0], cref)
    L.free()


@pytest.mark.parametrize("rep", [1, 2, 3, 4, 8])
def test_paired_kernel_every_rep(rep, monkeypatch):
    """The paired kernel streams rep value heads per key head with a two-deep
    prefetch: odd and even rep, rep = 1 (no prefetch) and the maximum."""
    monkeypatch.setenv("OMH_DECODE_KERNEL", "paired")
    d = GdnDims(2, 2 * rep, 64, 64, 4, 0)
    seed = 110 + rep
    w = synth.layer_weights(d, seed, gnorm_std=0.2, projections=False)
    B, T = 2, 3
    inp = synth.core_inputs(d, T, seed, B=B)
    conv0, S0 = synth.states(d, seed, B=B)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=B)
    for s in range(B):
        L.set_state(s, conv0[s], S0[s])
    got = np.stack([L.decode_core(inp["qkv"][:, t], inp["z"][:, t], inp["a"][:, t], inp["b"][:, t])
                    for t in range(T)], axis=1)
    for s in range(B):
        ref, cref, Sref = oracle.core_seq(d, w, inp["qkv"][s], inp["z"][s], inp["a"][s], inp["b"][s],
                                          conv0[s], S0[s])
        conv, S = L.get_state(s)
        assert_close(got[s], ref, what=f"rep={rep} seq {s} core")
        assert_close(S, Sref, what=f"rep={rep} seq {s} S")
        assert np.array_equal(conv, cref)
    L.free()


def test_paired_kernel_rejects_rep_above_limit(monkeypatch):
    monkeypatch.setenv("OMH_DECODE_KERNEL", "paired")
    d = GdnDims(1, 16, 16, 16, 4, 0)
    w = synth.layer_weights(d, 120, projections=False)
    L = gdn.GdnLayer(new_li(), d, w)
    inp = synth.core_inputs(d, 1, 120)
    with pytest.raises(gdn.OmhError) as e:
        L.decode_core(inp["qkv"], inp["z"], inp["a"], inp["b"])
    assert e.value.code == gdn.OMH_ERR_DEVICE
    monkeypatch.delenv("OMH_DECODE_KERNEL")
    core = L.decode_core(inp["qkv"], inp["z"], inp["a"], inp["b"])    # auto: sliced
    ref, _, _ = oracle.core_seq(d, w, inp["qkv"], inp["z"], inp["a"], inp["b"],
                                np.zeros((d.conv_dim, 3), np.float32), np.zeros((16, 16, 16), np.float32))
    assert_close(core, ref)
    L.free()


@pytest.mark.parametrize("B", [1, 2])
def test_decode_core_dev_30_layers_35b_vs_oracle(B):
    """Config 2's launch itself: the cores of 30 GDN layers of the 35B-A3B
    shape in one omh_gdn_decode_core_dev call, two steps, every layer's
    output, state and conv history against its own oracle run."""
    from overhang_amd import hip
    d = Q35B
    nl, T = 30, 2
    lays, ws, st0 = [], [], []
    for l in range(nl):
        w = synth.layer_weights(d, 500 + l, gnorm_std=0.1, projections=False)
        conv0, S0 = synth.states(d, 500 + l, B=B)
        L = gdn.GdnLayer(new_li(), d, w, max_seqs=B)
        for s in range(B):
            L.set_state(s, conv0[s], S0[s])
        lays.append(L)
        ws.append(w)
        st0.append((conv0, S0))
    inp = [synth.core_inputs(d, T, 600 + l, B=B) for l in range(nl)]     # per layer [B][T][...]
    core = hip.Buffer(nl * B * d.val_dim * 4)
    st = hip.Stream()
    got = np.empty((T, nl, B, d.val_dim), np.float32)
    for t in range(T):
        host = {k: np.ascontiguousarray(np.stack([inp[l][k][:, t] for l in range(nl)]))
                for k in ("qkv", "z", "a", "b")}
        dev = {k: hip.Buffer.from_numpy(v) for k, v in host.items()}
        gdn.decode_core_dev([L.li for L in lays], B, dev["qkv"], dev["z"], dev["a"], dev["b"], core,
                            stream=st)
        st.synchronize()
        got[t] = core.numpy((nl, B, d.val_dim))
    for l in range(nl):
        for s in range(B):
            ref, cref, Sref = oracle.core_seq(d, ws[l], inp[l]["qkv"][s], inp[l]["z"][s], inp[l]["a"][s],
                                              inp[l]["b"][s], st0[l][0][s], st0[l][1][s])
            conv, S = lays[l].get_state(s)
            assert_close(got[:, l, s], ref, what=f"layer {l} seq {s} core")
            assert_close(S, Sref, what=f"layer {l} seq {s} S")
            assert np.array_equal(conv, cref), f"layer {l} seq {s} conv history"
    for L in lays:
        L.free()


def test_decode_core_seq_dev_30_layers_rotating_slots():
    """The headline's launch: the cores of 30 GDN layers of the 35B-A3B shape
    stepping one sequence slot per call (omh_gdn_decode_core_seq_dev, B = 1,
    seq0 in a rotating order), so each call touches one slot's state in
    every layer and leaves the other slots (and their ring phases) alone.
    Every (layer, slot) output, final state and conv history against the
    oracle run over that slot's own tokens in order."""
    from overhang_amd import hip
    d = Q35B
    nl, S = 30, 4
    order = [0, 2, 1, 2, 3, 0, 2]
    lays, ws, st0 = [], [], []
    for l in range(nl):
        w = synth.layer_weights(d, 700 + l, gnorm_std=0.1, projections=False)
        conv0, S0 = synth.states(d, 700 + l, B=S)
        L = gdn.GdnLayer(new_li(), d, w, max_seqs=S)
        for s in range(S):
            L.set_state(s, conv0[s], S0[s])
        lays.append(L)
        ws.append(w)
        st0.append((conv0, S0))
    T = len(order)
    inp = [synth.core_inputs(d, T, 800 + l, B=1) for l in range(nl)]      # per layer [1][T][...]
    core = hip.Buffer(nl * d.val_dim * 4)
    st = hip.Stream()
    got = {}
    for t, s in enumerate(order):
        dev = {k: hip.Buffer.from_numpy(np.ascontiguousarray(np.stack([inp[l][k][0, t] for l in range(nl)])))
               for k in ("qkv", "z", "a", "b")}
        gdn.decode_core_seq_dev([L.li for L in lays], s, 1, dev["qkv"], dev["z"], dev["a"], dev["b"], core, stream=st)
        st.synchronize()
        got[t] = core.numpy((nl, d.val_dim))
    for s in range(S):
        ts = [t for t, q in enumerate(order) if q == s]
        for l in (0, 13, 29):
            conv, Sst = lays[l].get_state(s)
            if not ts:
                assert np.array_equal(Sst, st0[l][1][s]) and np.array_equal(conv, st0[l][0][s])
                continue
            ref, cref, Sref = oracle.core_seq(d, ws[l], *(inp[l][k][0, ts] for k in ("qkv", "z", "a", "b")),
                                              st0[l][0][s], st0[l][1][s])
            assert_close(np.stack([got[t][l] for t in ts]), ref, what=f"layer {l} slot {s} core")
            assert_close(Sst, Sref, what=f"layer {l} slot {s} S")
            assert np.array_equal(conv, cref), f"layer {l} slot {s} conv history"
    for L in lays:
        L.free()
