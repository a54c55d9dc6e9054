"""Decode steps captured in a HIP graph and replayed (the use the
allocation-free entry point serves, and how bench.py issues its engine-order
figures).

Layer chain: each layer's output is the next one's input, two tokens per
graph (so every layer's ring epoch alternates as in eager use).  A twin set
of layers runs the same tokens eagerly through omh_gdn_decode_dev.  The
graph is replayed three times with eager work and synchronisations in
between, and every replay's outputs, and the final states, must equal the
eager run's bit for bit (same kernels, same data)."""
import numpy as np
import pytest

from overhang_amd import gdn, hip, synth
from overhang_amd.dims import CFG1, Q35B

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,B,int8,nl", [(Q35B, 1, True, 3), (CFG1, 6, False, 4)], ids=["35b-int8-B1", "cfg1-B6"])
def test_graph_replays_equal_eager_decode(d, B, int8, nl):
    seed = 6100 + B
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed, B=B)
    base = 3400 + 20 * int8
    A = [gdn.GdnLayer(base + l, d, w, max_seqs=B, int8=int8) for l in range(nl)]
    E = [gdn.GdnLayer(base + 10 + l, d, w, max_seqs=B, int8=int8) for l in range(nl)]
    for L in A + E:
        for s in range(B):
            L.set_state(s, conv0[s], S0[s])
    st = hip.Stream()
    nbytes = B * d.hidden * 4
    xs = [hip.Buffer.from_numpy(synth.normal(seed + t, synth.S_X, (B, d.hidden))) for t in range(2)]
    ga = [[hip.Buffer(nbytes) for _ in range(nl)] for _ in range(2)]
    ea = [[hip.Buffer(nbytes) for _ in range(nl)] for _ in range(2)]

    def run(layers, outs, call):
        for t in range(2):
            for l in range(nl):
                call(layers[l].li, B, xs[t] if l == 0 else outs[t][l - 1], outs[t][l], stream=st)

    g = hip.Graph(st, lambda: run(A, ga, gdn.decode_noalloc_dev))
    try:
        assert g.nodes >= 2 * nl
        for rep in range(3):
            g.launch()
            st.synchronize()
            run(E, ea, gdn.decode_dev)                    # eager work between replays
            st.synchronize()
            for t in range(2):
                for l in range(nl):
                    a = ga[t][l].numpy((B, d.hidden))
                    e = ea[t][l].numpy((B, d.hidden))
                    assert np.isfinite(e).all()
                    np.testing.assert_array_equal(a, e, err_msg=f"replay {rep} token {t} layer {l}")
        for l in range(nl):
            for s in range(B):
                c1, S1 = A[l].get_state(s)
                c2, S2 = E[l].get_state(s)
                assert np.array_equal(c1, c2) and np.array_equal(S1, S2), f"layer {l} seq {s} state"
    finally:
        g.close()
        for L in A + E:
            L.free()
