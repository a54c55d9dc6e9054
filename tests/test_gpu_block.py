"""GPU parity of the whole GDN block (in_proj -> core -> out_proj) through the C-ABI.

The reference runs one token of one sequence per deltanet_step call
(overhang engines/qwen.c:301-364), with the projections as matvec /
matmul_q (qwen.c:70-77, 94-122).  Batched decode (B sequences, one token
each) and prefill (T tokens) must equal that per-token, per-sequence
recurrence (the CPU oracle) for every batch size, which covers both
projection kernels (register GEMV for up to 4 tokens, fp32 MFMA above) and
partial token tiles.  Tolerance: tests/tol.py."""
import numpy as np
import pytest

import oracle
from overhang_amd import gdn, synth
from overhang_amd.dims import CFG1, TINY, Q35B
from tests.tol import assert_close

pytestmark = pytest.mark.gpu

_next_li = [800]


def new_li():
    _next_li[0] += 1
    return _next_li[0]


def _x(d, seed, shape):
    return synth.normal(seed, synth.S_X, shape + (d.hidden,), 0.0, 1.0)


@pytest.mark.parametrize("dims,int8", [(CFG1, False), (TINY, True)], ids=["cfg1-f32", "tiny-int8"])
@pytest.mark.parametrize("B", [1, 2, 3, 4, 5, 17, 64])
def test_batched_decode_block_matches_oracle(dims, int8, B):
    d = dims
    seed = 9000 + B + 100 * int8
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed, B=B)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=B, int8=int8)
    for s in range(B):
        L.set_state(s, conv0[s], S0[s])
    T = 2
    x = _x(d, seed, (T, B))
    got = np.stack([L.decode(x[t]) for t in range(T)], axis=1)       # [B][T][D]
    for s in sorted({0, B // 2, B - 1}):
        ref, cref, Sref = oracle.layer_seq(d, w, x[:, s], conv0[s], S0[s], int8=int8)
        conv, S = L.get_state(s)
        assert_close(got[s], ref, what=f"B={B} seq {s} out")
        assert_close(S, Sref, what=f"B={B} seq {s} S")
        assert_close(conv, cref, atol=1e-5, rtol=1e-5, what=f"B={B} seq {s} conv")
    L.free()


@pytest.mark.parametrize("T", [5, 64, 65, 200, 300])
def test_prefill_block_matches_oracle(T):
    d = CFG1
    seed = 9500 + T
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed)
    for int8 in (False, True):
        L = gdn.GdnLayer(new_li(), d, w, int8=int8)
        L.set_state(0, conv0, S0)
        x = _x(d, seed, (T,))
        out = L.prefill(0, x)
        ref, cref, Sref = oracle.layer_seq(d, w, x, conv0, S0, int8=int8)
        conv, S = L.get_state(0)
        assert_close(out, ref, what=f"T={T} int8={int8} out")
        assert_close(S, Sref, what=f"T={T} int8={int8} S")
        L.free()


def test_35b_int8_block_batch64():
    """Qwen3.6-35B-A3B GDN block with int8 in/out projections (config 5
    shape): 64 sequences, one token each, three sequences checked."""
    d = Q35B
    B = 64
    w = synth.layer_weights(d, 77, gnorm_std=0.1)
    conv0, S0 = synth.states(d, 77, B=B)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=B, int8=True)
    for s in range(B):
        L.set_state(s, conv0[s], S0[s])
    x = _x(d, 77, (B,))
    got = L.decode(x)
    for s in (0, 31, 63):
        ref, cref, Sref = oracle.layer_seq(d, w, x[s:s + 1], conv0[s], S0[s], int8=True)
        conv, S = L.get_state(s)
        assert_close(got[s:s + 1], ref, what=f"seq {s} out")
        assert_close(S, Sref, what=f"seq {s} S")
    L.free()


@pytest.mark.parametrize("shape,B", [
    ((2, 4, 64, 64, 512), 5),        # sliced core kernel; out_proj on the staged bf16 x 3 kernel
    ((2, 4, 64, 64, 512), 40),
    ((4, 8, 128, 128, 1024), 64),    # paired core kernel; out_proj on the streaming kernel, k split over 2
    ((16, 32, 128, 128, 2048), 8),   # the 35B shape, sliced core; out_proj with a k split
], ids=["d64-B5", "d64-B40", "d128-B64", "35b-B8"])
def test_int8_block_core_writes_out_proj_planes(shape, B):
    """int8 blocks whose decode core also writes out_proj's x planes (int8
    planes with 128-wide block scales where the head width is a multiple of
    128, else bf16 planes and block sums), so the projection skips its split
    launch: two steps, three sequences against the per-token oracle."""
    from overhang_amd.dims import GdnDims
    kh, vh, kd, vd, hidden = shape
    d = GdnDims(kh=kh, vh=vh, kd=kd, vd=vd, K=4, hidden=hidden)
    seed = 9700 + B + kd
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed, B=B)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=B, int8=True)
    for s in range(B):
        L.set_state(s, conv0[s], S0[s])
    T = 2
    x = _x(d, seed, (T, B))
    got = np.stack([L.decode(x[t]) for t in range(T)], axis=1)       # [B][T][D]
    for s in sorted({0, B // 2, B - 1}):
        ref, cref, Sref = oracle.layer_seq(d, w, x[:, s], conv0[s], S0[s], int8=True)
        conv, S = L.get_state(s)
        assert_close(got[s], ref, what=f"{shape} B={B} seq {s} out")
        assert_close(S, Sref, what=f"{shape} B={B} seq {s} S")
    L.free()


def test_projection_shape_limits_are_reported():
    from overhang_amd.dims import GdnDims
    d = GdnDims(kh=2, vh=4, kd=16, vd=16, K=4, hidden=96)       # hidden not a multiple of 64
    w = synth.layer_weights(d, 1)
    with pytest.raises(gdn.OmhError) as e:
        gdn.GdnLayer(new_li(), d, w)
    assert e.value.code == gdn.OMH_ERR_SHAPE


@pytest.mark.parametrize("B,int8", [(1, True), (3, True), (1, False)], ids=["B1-int8", "B3-int8", "B1-f32"])
def test_35b_block_drop_in_small_batch(B, int8):
    """The engine's own call at the real shape: omh_gdn_decode(li, B, x, out)
    with the 35B-A3B GDN weights.  Up to 4 tokens the projections run on the
    register GEMV, whose k split is 2 for in_proj (I = 2048: 12288 int8 rows
    plus 64 fp32 b/a rows in one launch) and 4 for out_proj (I = 4096); with
    int8 rows the core runs as 4 column slices per value head and out_proj's
    GEMV applies the gated norm's 1 / rms.  Three tokens per sequence, each
    sequence against its own oracle run."""
    d = Q35B
    seed = 7100 + B + 10 * int8
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed, B=B)
    L = gdn.GdnLayer(new_li(), d, w, max_seqs=B, int8=int8)
    for s in range(B):
        L.set_state(s, conv0[s], S0[s])
    T = 3
    x = _x(d, seed, (T, B))
    got = np.stack([L.decode(x[t]) for t in range(T)], axis=1)       # [B][T][D]
    for s in range(B):
        ref, cref, Sref = oracle.layer_seq(d, w, x[:, s], conv0[s], S0[s], int8=int8)
        conv, S = L.get_state(s)
        assert_close(got[s], ref, what=f"35B B={B} int8={int8} seq {s} out")
        assert_close(S, Sref, what=f"35B B={B} int8={int8} seq {s} S")
        # the history holds in_proj outputs: a floating-point result here
        assert_close(conv, cref, what=f"35B B={B} int8={int8} seq {s} conv")
    L.free()


@pytest.mark.parametrize("shape,B", [(None, 1), (None, 2), (None, 3), (None, 4),
                                     ((2, 4, 64, 64, 512), 1), ((2, 4, 64, 64, 512), 4)],
                         ids=["35b-B1", "35b-B2", "35b-B3", "35b-B4", "d64-B1", "d64-B4"])
def test_deferred_norm_matches_norm_in_core(shape, B, monkeypatch):
    """At up to 4 tokens with int8 out_proj rows the decode core runs as 4
    column slices per value head, each writing o * gnorm * silu(z) and its
    sum of squares of o, and out_proj's GEMV applies each head's 1 / rms as
    it loads x.  With OMH_DECODE_KERNEL=sliced and OMH_DECODE_NCS=1 the same
    call keeps one workgroup per value head with the whole gated norm in the
    core.  Only the order of fp32 sums and products differs between the two,
    so they agree far inside the oracle contract: outputs within 2e-5
    relative, states and conv histories within 1e-5 (a head or slice mixed
    up would be off by the norm itself).  Both are also held to the oracle.
    The 35B shape (slices of 32 columns, out_proj k = 4096) and 64-wide
    heads (slices of 16 columns: one GEMV input piece each)."""
    from overhang_amd.dims import GdnDims
    d = Q35B if shape is None else GdnDims(kh=shape[0], vh=shape[1], kd=shape[2], vd=shape[3], K=4, hidden=shape[4])
    seed = 7150 + B + (0 if shape is None else 40)
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed, B=B)
    La = gdn.GdnLayer(new_li(), d, w, max_seqs=B, int8=True)
    Lb = gdn.GdnLayer(new_li(), d, w, max_seqs=B, int8=True)
    try:
        for s in range(B):
            La.set_state(s, conv0[s], S0[s])
            Lb.set_state(s, conv0[s], S0[s])
        T = 3
        x = _x(d, seed, (T, B))
        ya_all = []
        for t in range(T):
            ya = La.decode(x[t])
            monkeypatch.setenv("OMH_DECODE_KERNEL", "sliced")
            monkeypatch.setenv("OMH_DECODE_NCS", "1")
            yb = Lb.decode(x[t])
            monkeypatch.delenv("OMH_DECODE_KERNEL")
            monkeypatch.delenv("OMH_DECODE_NCS")
            err = float(np.abs(ya - yb).max())
            print(f"{d.kd}/{d.vd} B={B} token {t}: max |deferred - in-core| = {err:.3g} (max |out| {float(np.abs(yb).max()):.3g})")
            np.testing.assert_allclose(ya, yb, rtol=2e-5, atol=1e-6 * float(np.abs(yb).max()), err_msg=f"token {t}")
            ya_all.append(ya)
        got = np.stack(ya_all, axis=1)                                    # [B][T][D]
        for s in range(B):
            ca, Sa = La.get_state(s)
            cb, Sb = Lb.get_state(s)
            np.testing.assert_allclose(Sa, Sb, rtol=1e-5, atol=1e-6, err_msg=f"seq {s} S")
            np.testing.assert_allclose(ca, cb, rtol=1e-5, atol=1e-6, err_msg=f"seq {s} conv")
            ref, cref, Sref = oracle.layer_seq(d, w, x[:, s], conv0[s], S0[s], int8=True)
            assert_close(got[s], ref, what=f"deferred {d.kd}/{d.vd} B={B} seq {s} out")
            assert_close(Sa, Sref, what=f"deferred {d.kd}/{d.vd} B={B} seq {s} S")
    finally:
        La.free()
        Lb.free()


@pytest.mark.parametrize("T", [65, 128, 255, 256, 333, 1024])
def test_35b_int8_prefill_block_matches_oracle(T):
    """Row f2 at prefill size: the 35B-A3B int8 layer through
    omh_gdn_prefill, whose int8 projections (in_proj 2048 -> 12352 with the
    fp32 b/a rows beside, out_proj 4096 -> 2048) run on the int8 wave-tile
    kernel for 65..255 tokens and on the int8 matrix-core GEMM from 256
    tokens (T = 65, 255, 333: partial token tiles), continuing from a
    nonzero state.  Every token's output and the final state and conv
    history are compared with the per-token oracle (engines/qwen.c:301-364
    with matmul_q, qwen.c:94-122)."""
    d = Q35B
    seed = 7300 + T
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed)
    L = gdn.GdnLayer(new_li(), d, w, int8=True)
    L.set_state(0, conv0, S0)
    x = _x(d, seed, (T,))
    out = L.prefill(0, x)
    ref, cref, Sref = oracle.layer_seq(d, w, x, conv0, S0, int8=True)
    conv, S = L.get_state(0)
    assert_close(out, ref, what=f"35B int8 prefill T={T} out")
    assert_close(S, Sref, what=f"35B int8 prefill T={T} S")
    assert_close(conv, cref, what=f"35B int8 prefill T={T} conv")
    # a decode step after the prefill continues the same recurrence
    x1 = _x(d, seed + 1, (1,))
    o1 = L.decode(x1)
    ref1, _, Sref1 = oracle.layer_seq(d, w, x1, cref, Sref, int8=True)
    assert_close(o1, ref1, what="decode after prefill out")
    assert_close(L.get_state(0)[1], Sref1, what="decode after prefill S")
    L.free()


@pytest.mark.parametrize("shape,T", [((16, 32, 128, 128, 2048), 300), ((3, 6, 64, 64, 1024), 270)],
                         ids=["35b-T300", "kh3-T270"])
def test_int8_gemm_matches_wave_kernel(shape, T, monkeypatch):
    """The prefill-sized int8 GEMM against the int8 wave-tile kernel it
    replaces from 256 tokens (OMH_I8_GEMM forces either): both sum every
    plane product exactly in int32, so the two layers agree to fp32
    rounding of the plane combine (kh3: 1152 in_proj int8 rows, not a
    multiple of the GEMM's 256-row tile; both: partial token tiles)."""
    from overhang_amd.dims import GdnDims
    kh, vh, kd, vd, hidden = shape
    d = GdnDims(kh=kh, vh=vh, kd=kd, vd=vd, K=4, hidden=hidden)
    seed = 7600 + T
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed)
    x = _x(d, seed, (T,))
    outs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("OMH_I8_GEMM", mode)
        L = gdn.GdnLayer(new_li(), d, w, int8=True)
        L.set_state(0, conv0, S0)
        outs[mode] = (L.prefill(0, x), L.get_state(0)[1])
        L.free()
    assert_close(outs["1"][0], outs["0"][0], atol=2e-5, rtol=2e-5, what=f"{T} gemm vs wave out")
    assert_close(outs["1"][1], outs["0"][1], atol=2e-5, rtol=2e-5, what=f"{T} gemm vs wave S")


@pytest.mark.parametrize("shape,B", [((16, 32, 128, 128, 2048), 64), ((16, 32, 128, 128, 2048), 17),
                                     ((3, 6, 64, 64, 1024), 40)],
                         ids=["35b-B64", "35b-B17", "kh3-B40"])
def test_int8_decode_batch_kernel_matches_stream_kernel(shape, B, monkeypatch):
    """The split-queue int8 kernel for decode batches of 5..64 tokens (one
    set of waves copies the tiled weights into LDS, the other loads x and
    runs the products) against the streaming kernel it replaces
    (OMH_I8_DQ=0): both sum the plane products exactly in int32, so two
    decode steps agree to fp32 rounding (B = 17: a partial token tile;
    kh3: 1152 in_proj int8 rows, not a multiple of the 64-row workgroup
    tile).  test_35b_int8_block_batch64 pins the same kernel to the oracle."""
    from overhang_amd.dims import GdnDims
    kh, vh, kd, vd, hidden = shape
    d = GdnDims(kh=kh, vh=vh, kd=kd, vd=vd, K=4, hidden=hidden)
    seed = 7800 + B
    w = synth.layer_weights(d, seed, gnorm_std=0.1)
    conv0, S0 = synth.states(d, seed, B=B)
    x = _x(d, seed, (2, B))
    outs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("OMH_I8_DQ", mode)
        L = gdn.GdnLayer(new_li(), d, w, max_seqs=B, int8=True)
        for s in range(B):
            L.set_state(s, conv0[s], S0[s])
        o = np.stack([L.decode(x[t]) for t in range(2)])
        outs[mode] = (o, np.stack([L.get_state(s)[1] for s in (0, B - 1)]))
        L.free()
    assert_close(outs["1"][0], outs["0"][0], atol=2e-5, rtol=2e-5, what=f"B={B} split-queue vs stream out")
    assert_close(outs["1"][1], outs["0"][1], atol=2e-5, rtol=2e-5, what=f"B={B} split-queue vs stream S")
