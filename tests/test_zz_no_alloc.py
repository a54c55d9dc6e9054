"""omh_gdn_decode_noalloc_dev: the allocation-free variant of
omh_gdn_decode_dev (its scratch is the library's static 8 MiB device buffer).

Two layers with identical weights and states: one driven through
omh_gdn_decode_dev, the other through the no-alloc entry point, the same
inputs.  Two calls in a row, the second with a smaller batch (and a second
round with the order of sizes that takes the other projection paths): the
outputs and the states must be identical, since both run the same kernels
on the same data.  A batch whose scratch exceeds the static buffer is
refused with OMH_ERR_SHAPE before anything runs."""
import numpy as np
import pytest

from overhang_amd import gdn, hip, synth
from overhang_amd.dims import Q35B, CFG1

pytestmark = pytest.mark.gpu


def _pair(d, seed, B, int8, li0):
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed, B=B)
    L1 = gdn.GdnLayer(li0, d, w, max_seqs=B, int8=int8)
    L2 = gdn.GdnLayer(li0 + 1, d, w, max_seqs=B, int8=int8)
    for s in range(B):
        L1.set_state(s, conv0[s], S0[s])
        L2.set_state(s, conv0[s], S0[s])
    return L1, L2


@pytest.mark.parametrize("d,int8,sizes", [
    (Q35B, True, (64, 3)),        # split-queue in_proj, paired core in two launches, streaming out_proj; then the GEMVs
                                  # around a column-sliced core whose 1 / rms out_proj applies
    (Q35B, True, (17, 8)),        # partial token tiles (17 = 16 + 1), then a sliced-kernel core at B = 8
    (CFG1, False, (40, 1)),       # fp32 MFMA projections, then the GEMV
], ids=["35b-int8-64-3", "35b-int8-17-8", "cfg1-f32-40-1"])
def test_noalloc_decode_equals_decode_dev(d, int8, sizes):
    B = max(sizes)
    L1, L2 = _pair(d, 4400 + B, B, int8, 3200 + 2 * B + int8)
    st = hip.Stream()
    try:
        for call, b in enumerate(sizes):
            x = hip.Buffer.from_numpy(synth.normal(4500 + call, synth.S_X, (b, d.hidden)))
            o1, o2 = hip.Buffer(b * d.hidden * 4), hip.Buffer(b * d.hidden * 4)
            gdn.decode_dev(L1.li, b, x, o1, stream=st)
            gdn.decode_noalloc_dev(L2.li, b, x, o2, stream=st)
            st.synchronize()
            r1, r2 = o1.numpy((b, d.hidden)), o2.numpy((b, d.hidden))
            print(f"call {call}: B={b} max |noalloc - dev| = {float(np.abs(r1 - r2).max()):.3g}")
            np.testing.assert_array_equal(r2, r1, err_msg=f"call {call} B={b}")
        for s in range(B):
            c1, S1 = L1.get_state(s)
            c2, S2 = L2.get_state(s)
            assert np.array_equal(c1, c2) and np.array_equal(S1, S2), f"seq {s} state"
    finally:
        L1.free()
        L2.free()


def test_noalloc_rejects_batches_beyond_its_buffer():
    """35B int8 at B = 512: the in_proj rows alone need 25 MB > 8 MiB."""
    d = Q35B
    L = gdn.GdnLayer(3490, d, synth.layer_weights(d, 4490), max_seqs=512, int8=True)
    x = hip.Buffer(512 * d.hidden * 4)
    o = hip.Buffer(512 * d.hidden * 4)
    try:
        with pytest.raises(gdn.OmhError) as e:
            gdn.decode_noalloc_dev(L.li, 512, x, o)
        assert e.value.code == gdn.OMH_ERR_SHAPE and "static buffer" in str(e.value)
    finally:
        L.free()
