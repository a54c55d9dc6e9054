"""GPU parity of the gated full-attention layer (engines/qwen.c:366-425,
attn_step) through the C-ABI (omh_attn_forward).

The checker is tests/qwen_tiny.gated_attention, the float32 restatement of
attn_step that the host model runs; with it the host model reproduces the
reference's own golden tokens (greedy `full_ids` 20/20, teacher-forced
`tf_argmax` 28/28, test_e2e_tiny.py), and the closed-form cases in
test_attn_ref.py pin its parts.  Here the GPU layer must match it:
  - on the reference tiny model, as the model's attention layers, to the
    same golden tokens (GDN layers on the GPU as well);
  - at the Qwen3.6-35B-A3B attention shape (hidden 2048, 16 query heads,
    2 kv heads, head_dim 256, rot 64) through prompt steps (one key split)
    and decode steps (up to 47 key splits of 64 keys);
  - over the other head widths and group sizes the kernels take, int8
    projections, several sequences, and the argument checks.
Tolerance: tests/tol.py (max-abs 2e-3 / rel 1e-3)."""
import numpy as np
import pytest

from overhang_amd import gdn
from tests import qwen_tiny as q
from tests.tol import assert_close

pytestmark = pytest.mark.gpu

_next = [1200]


def new_li():
    _next[0] += 1
    return _next[0]


def _weights(rng, D, H, KV, hd, scale=0.02):
    return {"W_q": rng.normal(0, scale, (2 * H * hd, D)).astype(np.float32),
            "W_k": rng.normal(0, scale, (KV * hd, D)).astype(np.float32),
            "W_v": rng.normal(0, scale, (KV * hd, D)).astype(np.float32),
            "W_o": rng.normal(0, scale, (D, H * hd)).astype(np.float32),
            "q_norm": rng.normal(0, 0.1, hd).astype(np.float32),
            "k_norm": rng.normal(0, 0.1, hd).astype(np.float32)}


def _ref_w(w):
    return {"q_proj": w["W_q"], "k_proj": w["W_k"], "v_proj": w["W_v"], "o_proj": w["W_o"],
            "q_norm": w["q_norm"], "k_norm": w["k_norm"]}


def _dequant(w):
    """The weights the int8 path computes with: q * s per row (qwen.c:116-121)."""
    out = dict(w)
    for nm in ("q", "k", "v", "o"):
        Q, S = gdn.quantize_rows(w["W_" + nm])
        out["W_" + nm] = (Q.astype(np.float32) * S[:, None]).astype(np.float32)
    return out


def _run(shape, steps, seed=0, int8=False, max_t=None, x_scale=1.0):
    """steps: token counts of consecutive calls on sequence 0."""
    D, H, KV, hd, rot = shape
    rng = np.random.default_rng(seed)
    w = _weights(rng, D, H, KV, hd)
    total = sum(steps)
    L = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, max_t or total, w, int8=int8)
    rw = _ref_w(_dequant(w) if int8 else w)
    Kl, Vl = [], []
    pos = 0
    try:
        for T in steps:
            x = (rng.normal(0, 1, (T, D)) * x_scale).astype(np.float32)
            got = L.forward(0, pos, x)
            ref = q.gated_attention(x, rw, Kl, Vl, pos, H, KV, hd, rot, 1e7, 1e-6)
            assert_close(got, ref, what=f"shape {shape} pos {pos} T {T}")
            pos += T
    finally:
        L.free()


Q35B_ATTN = (2048, 16, 2, 256, 64)


def test_tiny_greedy_with_gpu_attention_and_gdn():
    m = q.TinyQwen(q.HipGdn, first_li=960, gpu_attn_li=1100)
    try:
        got, exp = q.greedy(m)
    finally:
        m.close()
    assert got == exp, f"greedy {sum(int(a == b) for a, b in zip(got, exp))}/20: {got} vs {exp}"


def test_tiny_teacher_forced_with_gpu_attention_prompt_step():
    """All 28 positions in one forward: each attention layer is one T = 28
    call, each GDN layer one chunked prefill."""
    m = q.TinyQwen(q.HipGdn, first_li=980, batched=True, gpu_attn_li=1150)
    try:
        got, exp = q.teacher_forced(m)
    finally:
        m.close()
    assert got == exp, f"teacher-forced {sum(int(a == b) for a, b in zip(got, exp))}/28"


@pytest.mark.parametrize("steps", [[1, 1, 1], [37, 1, 1], [200, 1, 64, 1], [37, 100, 1, 71]],
                         ids=["decode", "prompt37", "prompt200", "prompt-after-prompt"])
def test_35b_shape_prompt_then_decode(steps):
    """Prompt steps of 64 tokens and more run on a flash kernel (the
    default bf16 x 3 one, three bf16 products per fp32 product, and the
    fp32-product one that OMH_ATTN_FLASH=fp32 selects), shorter ones and
    decode steps on the split kernel; a prompt step may start after earlier
    tokens (pos > 0)."""
    _run(Q35B_ATTN, steps)


@pytest.mark.parametrize("steps", [[200, 1, 64, 1], [37, 100, 1, 71]], ids=["prompt200", "prompt-after-prompt"])
def test_35b_shape_prompt_then_decode_fp32_flash(steps, monkeypatch):
    """The same sequences with prompt steps on the fp32-product flash kernel."""
    monkeypatch.setenv("OMH_ATTN_FLASH", "fp32")
    _run(Q35B_ATTN, steps)


def test_35b_shape_long_context_many_splits():
    """A 3000-token prompt in one call, then decode steps at n = 3001..3003:
    47 key splits of 64 keys per kv head."""
    _run(Q35B_ATTN, [3000, 1, 1, 1], seed=3)


@pytest.mark.parametrize("shape", [(256, 8, 8, 32, 32), (128, 4, 1, 64, 16), (512, 16, 1, 128, 128),
                                   (256, 2, 2, 128, 0), (1024, 4, 4, 256, 256)],
                         ids=["hd32-grp1", "hd64-grp4", "hd128-grp16", "hd128-norope", "hd256-fullrope"])
def test_head_widths_and_groups(shape):
    _run(shape, [70, 1, 5, 1], seed=7)


@pytest.mark.parametrize("steps", [[1, 1], [64, 1]], ids=["decode", "prompt64"])
def test_int8_projections(steps):
    _run(Q35B_ATTN, steps, seed=11, int8=True)


def test_sequences_are_isolated():
    D, H, KV, hd, rot = 256, 4, 2, 64, 16
    rng = np.random.default_rng(5)
    w = _weights(rng, D, H, KV, hd)
    L = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, 64, w, max_seqs=3)
    rw = _ref_w(w)
    try:
        caches = {s: ([], []) for s in (0, 2)}
        pos = {0: 0, 2: 0}
        for s, T in [(0, 10), (2, 7), (0, 1), (2, 3), (0, 1), (2, 1)]:
            x = rng.normal(0, 1, (T, D)).astype(np.float32)
            got = L.forward(s, pos[s], x)
            ref = q.gated_attention(x, rw, *caches[s], pos[s], H, KV, hd, rot, 1e7, 1e-6)
            assert_close(got, ref, what=f"seq {s} pos {pos[s]}")
            pos[s] += T
    finally:
        L.free()


def test_argument_checks():
    D, H, KV, hd, rot = 128, 2, 1, 64, 16
    rng = np.random.default_rng(1)
    w = _weights(rng, D, H, KV, hd)
    with pytest.raises(gdn.OmhError) as e:
        gdn.AttnLayer(new_li(), D, H, KV, 96, rot, 1e7, 1e-6, 8, _weights(rng, D, H, KV, 96))
    assert e.value.code == gdn.OMH_ERR_SHAPE
    L = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, 8, w)
    try:
        x = np.zeros((4, D), np.float32)
        with pytest.raises(gdn.OmhError):
            L.forward(0, 5, x)                   # positions 5..8 past max_t = 8
        with pytest.raises(gdn.OmhError):
            L.forward(1, 0, x)                   # one sequence only
        assert L.forward(0, 4, x).shape == (4, D)
    finally:
        L.free()


def test_device_pointer_entry_matches_host_entry():
    """omh_attn_forward_dev on a library-external stream: the same results as
    the host entry point, bit for bit, over a prompt and decode steps."""
    from overhang_amd import hip
    D, H, KV, hd, rot = Q35B_ATTN
    rng = np.random.default_rng(21)
    w = _weights(rng, D, H, KV, hd)
    A = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, 128, w)
    B = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, 128, w)
    st = hip.Stream()
    try:
        pos = 0
        for T in (33, 1, 1):
            x = rng.normal(0, 1, (T, D)).astype(np.float32)
            xd, od = hip.Buffer.from_numpy(x), hip.Buffer(T * D * 4)
            gdn.attn_forward_dev(A.li, 0, pos, T, xd, od, stream=st)
            st.synchronize()
            np.testing.assert_array_equal(od.numpy((T, D)), B.forward(0, pos, x))
            pos += T
    finally:
        A.free()
        B.free()


def test_cache_get_waits_for_device_pointer_calls():
    """omh_attn_cache_get right after omh_attn_forward_dev on a caller's
    stream, with no synchronisation in between: the copy waits for the
    device (as omh_gdn_state_get does), so it returns the rows the step
    wrote, equal to those of the same step run through the host entry."""
    from overhang_amd import hip
    D, H, KV, hd, rot = Q35B_ATTN
    rng = np.random.default_rng(22)
    w = _weights(rng, D, H, KV, hd)
    T = 2048
    A = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, T, w)
    B = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, T, w)
    st = hip.Stream()
    try:
        x = rng.normal(0, 1, (T, D)).astype(np.float32)
        B.forward(0, 0, x)
        Kb, Vb = B.cache_get(0, 0, T)
        xd, od = hip.Buffer.from_numpy(x), hip.Buffer(T * D * 4)
        gdn.attn_forward_dev(A.li, 0, 0, T, xd, od, stream=st)
        Ka, Va = A.cache_get(0, 0, T)            # no st.synchronize() before it
        np.testing.assert_array_equal(Ka, Kb)
        np.testing.assert_array_equal(Va, Vb)
        st.synchronize()
    finally:
        A.free()
        B.free()


@pytest.mark.parametrize("name", ["attn_tiny_f32", "attn_tiny_int8", "attn_35b_f32", "attn_35b_int8"])
def test_attention_matches_reference_attn_golden(name):
    """The GPU layer against the reference's own attn_step (qwen.c:367-425,
    fixtures written by tests/golden/make_golden.py): the cache rows
    0..pos0-1 are seeded through omh_attn_cache_set, then the fixture's
    tokens run one call each at positions pos0.. (up to 8002, the 35B
    shape), and the written cache rows come back through
    omh_attn_cache_get."""
    from tests.test_attn_ref import load_attn
    s, w, x, Kpre, Vpre, exp = load_attn(name)
    D, H, KV, hd, rot, pos0, T = (s[k] for k in ("D", "H", "KV", "hd", "rot", "pos0", "T"))
    L = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, s["theta"], s["eps"], pos0 + T, w, int8=s["int8"])
    try:
        L.cache_set(0, 0, pos0, np.ascontiguousarray(Kpre.transpose(1, 0, 2)),
                    np.ascontiguousarray(Vpre.transpose(1, 0, 2)))
        got = np.concatenate([L.forward(0, pos0 + t, x[t:t + 1]) for t in range(T)])
        assert_close(got, exp["out"], what=f"{name} out")
        K, V = L.cache_get(0, pos0, T, pos0 + T)
        assert_close(K[:, pos0:].transpose(1, 0, 2), exp["K"], what=f"{name} K rows")
        assert_close(V[:, pos0:].transpose(1, 0, 2), exp["V"], what=f"{name} V rows")
        K0, _ = L.cache_get(0, 0, pos0, pos0 + T)
        assert np.array_equal(K0[:, :pos0], Kpre.transpose(1, 0, 2)), "seeded rows come back unchanged"
    finally:
        L.free()


def test_flash_bf16x3_matches_fp32_products(monkeypatch):
    """The bf16 x 3 flash kernel (the default for prompt steps) against the
    fp32-product flash kernel on the same 35B-shape prompt (OMH_ATTN_FLASH
    selects): three bf16 products per fp32 one leave a relative error near
    2^-16 per product, far inside the layer's tolerance."""
    D, H, KV, hd, rot = Q35B_ATTN
    rng = np.random.default_rng(23)
    w = _weights(rng, D, H, KV, hd)
    x = rng.normal(0, 1, (300, D)).astype(np.float32)
    outs = {}
    for mode in ("fp32", "bf16x3"):
        monkeypatch.setenv("OMH_ATTN_FLASH", mode)
        L = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, 300, w)
        try:
            outs[mode] = L.forward(0, 0, x)
        finally:
            L.free()
    assert_close(outs["bf16x3"], outs["fp32"], atol=2e-5, rtol=2e-4, what="flash bf16x3 vs fp32")


@pytest.mark.parametrize("shape,steps", [(Q35B_ATTN, [300]), (Q35B_ATTN, [37, 300]), ((512, 16, 1, 128, 128), [257])],
                         ids=["35b-T300", "35b-pos37-T300", "hd128-T257"])
def test_flash_tile_images_match_tiles_staged_in_kernel(shape, steps, monkeypatch):
    """Prompt steps of 256 tokens and more stage the bf16 x 3 flash kernel's
    tiles from images made once per call (attn_tile_image_kernel); the
    kernel converting every tile itself (OMH_ATTN_FLASH=reg) must give the
    same outputs and cache rows bit for bit: masked keys contribute exactly
    zero either way."""
    D, H, KV, hd, rot = shape
    rng = np.random.default_rng(31)
    w = _weights(rng, D, H, KV, hd)
    total = sum(steps)
    xs = [rng.normal(0, 1, (T, D)).astype(np.float32) for T in steps]
    res = {}
    for mode in ("reg", "img"):
        monkeypatch.delenv("OMH_ATTN_FLASH", raising=False)
        if mode == "reg":
            monkeypatch.setenv("OMH_ATTN_FLASH", "reg")
        L = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, total, w)
        try:
            pos, outs = 0, []
            for x in xs:
                outs.append(L.forward(0, pos, x))
                pos += x.shape[0]
            res[mode] = (np.concatenate(outs), L.cache_get(0, 0, total))
        finally:
            L.free()
    assert np.array_equal(res["img"][0], res["reg"][0]), "outputs differ"
    assert np.array_equal(res["img"][1][0], res["reg"][1][0]) and np.array_equal(res["img"][1][1], res["reg"][1][1])


@pytest.mark.parametrize("shape", [Q35B_ATTN, (256, 8, 8, 32, 32), (512, 16, 1, 128, 128), (1024, 4, 4, 256, 256)],
                         ids=["35b", "hd32-grp1", "hd128-grp16", "hd256-fullrope"])
def test_decode_prep_in_split_kernel_matches_prep_launch(shape, monkeypatch):
    """Decode steps form q, and the new k / v cache rows, inside the split
    kernel (the workgroup whose key split holds the position writes the
    rows); OMH_ATTN_FUSE=0 keeps the prep launch.  Same operations in the
    same order: the outputs and the cache rows are equal bit for bit, over
    decode steps at positions 62..65 after a 62-token prompt: the last rows
    of the first 64-key split and the first of the second."""
    D, H, KV, hd, rot = shape
    rng = np.random.default_rng(29)
    w = _weights(rng, D, H, KV, hd)
    xs = [rng.normal(0, 1, (62, D)).astype(np.float32)] + [rng.normal(0, 1, (1, D)).astype(np.float32) for _ in range(4)]
    outs = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("OMH_ATTN_FUSE", mode)
        L = gdn.AttnLayer(new_li(), D, H, KV, hd, rot, 1e7, 1e-6, 80, w)
        try:
            got, pos = [], 0
            for x in xs:
                got.append(L.forward(0, pos, x))
                pos += x.shape[0]
            K, V = L.cache_get(0, 0, 0, pos)
            outs[mode] = (np.concatenate(got), K, V)
        finally:
            L.free()
    for a, b, nm in zip(outs["1"], outs["0"], ("out", "K cache", "V cache")):
        np.testing.assert_array_equal(a, b, err_msg=f"{shape} fused prep vs prep launch: {nm}")
