"""Device-side GDN state snapshot and rollback for speculative decoding
(omh_gdn_state_copy), through the C-ABI.

The reference has no such operation (its worklog records deltanet rollback
as infeasible as implemented, WORKLOG.md:157-158; multi-token prediction is
on its roadmap, ROADMAP.md:10).  What fixes the result is the recurrence
itself: after snapshot -> speculative tokens -> rollback, a sequence must be
in exactly the state it had at the snapshot, so every later output must be
bit-identical to a run that never took the speculative tokens.  Checked for
the whole layer (projections + core) with decode steps, with a speculative
verify step run as a prefill, at the fp32 cfg1 shape and the 35B int8 shape;
speculation lengths 1..5 move the conv ring to every phase."""
import numpy as np
import pytest

from overhang_amd import gdn, synth
from overhang_amd.dims import CFG1, Q35B

pytestmark = pytest.mark.gpu

_next = [1400]


def new_li():
    _next[0] += 1
    return _next[0]


def _x(d, seed, T):
    return synth.normal(seed, synth.S_X, (T, d.hidden), 0.0, 1.0)


@pytest.mark.parametrize("d,int8,spec,verify_prefill",
                         [(CFG1, False, 1, False), (CFG1, False, 3, True), (CFG1, False, 4, False),
                          (Q35B, True, 5, True), (Q35B, True, 2, False)],
                         ids=["cfg1-s1", "cfg1-s3-prefill", "cfg1-s4", "35b-int8-s5-prefill", "35b-int8-s2"])
def test_rollback_equals_run_without_speculation(d, int8, spec, verify_prefill):
    w = synth.layer_weights(d, 3)
    A = gdn.GdnLayer(new_li(), d, w, max_seqs=2, int8=int8)
    B = gdn.GdnLayer(new_li(), d, w, max_seqs=1, int8=int8)
    x = _x(d, 4, 40)
    try:
        # a prompt, then two decode tokens, on both
        np.testing.assert_array_equal(A.prefill(0, x[:29]), B.prefill(0, x[:29]))
        for k in (29, 30):
            np.testing.assert_array_equal(A.decode(x[k:k + 1]), B.decode(x[k:k + 1]))
        A.copy_state(0, 1)                                   # snapshot into the spare slot
        snap = A.get_state(0)
        np.testing.assert_array_equal(A.get_state(1)[1], snap[1])
        draft = _x(d, 5, spec) * 0.5
        if verify_prefill:
            A.prefill(0, draft)                              # a verify step over the draft tokens
        else:
            for k in range(spec):
                A.decode(draft[k:k + 1])
        assert not np.array_equal(A.get_state(0)[1], snap[1])
        A.copy_state(1, 0)                                   # rollback
        conv, S = A.get_state(0)
        np.testing.assert_array_equal(conv, snap[0])
        np.testing.assert_array_equal(S, snap[1])
        for k in range(31, 36):
            np.testing.assert_array_equal(A.decode(x[k:k + 1]), B.decode(x[k:k + 1]), err_msg=f"token {k}")
        np.testing.assert_array_equal(A.prefill(0, x[36:40]), B.prefill(0, x[36:40]))
    finally:
        A.free()
        B.free()


def test_copy_argument_checks():
    d = CFG1
    L = gdn.GdnLayer(new_li(), d, synth.layer_weights(d, 1), max_seqs=2)
    try:
        for src, dst in ((0, 2), (-1, 0), (2, 1)):
            with pytest.raises(gdn.OmhError) as e:
                L.copy_state(src, dst)
            assert e.value.code == gdn.OMH_ERR_ARG
        L.copy_state(1, 1)                                   # a no-op
    finally:
        L.free()


def test_one_launch_over_many_layers_and_device_entry():
    """The multi-layer copy (40 layers: two launches of up to 32) through the
    device-pointer entry point on a stream: every layer's state moves."""
    from overhang_amd import hip
    d = CFG1
    w = synth.layer_weights(d, 2, projections=False)
    lays = [gdn.GdnLayer(new_li(), d, w, max_seqs=3) for _ in range(40)]
    st = hip.Stream()
    try:
        for i, L in enumerate(lays):
            conv, S = synth.states(d, 100 + i)
            L.set_state(2, conv, S)
        gdn.state_copy_dev([L.li for L in lays], 2, 0, stream=st)
        st.synchronize()
        for L in lays:
            c0, S0 = L.get_state(0)
            c2, S2 = L.get_state(2)
            np.testing.assert_array_equal(c0, c2)
            np.testing.assert_array_equal(S0, S2)
    finally:
        for L in lays:
            L.free()
