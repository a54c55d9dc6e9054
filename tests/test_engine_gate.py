"""The drop-in through the reference engine itself.

tests/engine/Makefile compiles the reference engines/qwen.c (read in place,
never copied) with the om_hip hooks of tests/engine/omh_qwen_hooks.h and
links it to overhang_amd/libom_hip.so.  These tests run that binary on the
reference's tiny model and its own gate (reference Makefile:34-35 ->
engines/qwen.c:616-658: exit 0 iff the greedy continuation matches
full_ids 20/20), plus the teacher-forced gate against tf_argmax (28/28)
through the batched prompt step the hooks add.

On the GPU the GDN and attention layers run in libom_hip.so (the engine says
so on stderr); with OM_HIP=0, or with no usable device, the same binary
keeps every layer on its CPU body."""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ENGINE = os.path.join(ROOT, "tests", "engine", "_build", "qwen_hip")
TINY = os.path.join(ROOT, "tests", "golden", "qwen_tiny")
REFJ = os.path.join(TINY, "ref_qwen.json")
ON_GPU = "om_hip: GDN and attention layers on the GPU"


def run(args, stdin=None, **env):
    if not os.path.exists(ENGINE):
        pytest.fail(f"{ENGINE} is not built: run __graft_entry__.build() where the reference sources are present")
    e = dict(os.environ, SNAP=TINY)
    for k in ("OM_HIP", "OMH_BATCH_PROMPT", "OMH_TEST_FAIL_LAYER"):
        e.pop(k, None)
    e.update(env)
    r = subprocess.run([ENGINE] + args, env=e, input=stdin, capture_output=True, text=True, timeout=300)
    print(r.stdout[-600:])
    print(r.stderr[-600:])
    return r


def test_engine_cpu_gate_with_om_hip_off():
    """OM_HIP=0: the reference engine's own body, greedy 20/20."""
    r = run([REFJ], OM_HIP="0")
    assert r.returncode == 0 and "greedy match: 20/20" in r.stdout, r.stdout[-300:]
    assert ON_GPU not in r.stderr


def test_engine_cpu_teacher_forced_gate_with_om_hip_off():
    r = run(["--tf", REFJ], OM_HIP="0")
    assert r.returncode == 0 and "teacher-forced match: 28/28" in r.stdout, r.stdout[-300:]


@pytest.mark.gpu
def test_engine_greedy_gate_gdn_and_attention_on_gpu():
    """The reference gate with every GDN layer as omh_gdn_decode(li, 1, x,
    out) and every attention layer as omh_attn_forward, one token per call."""
    r = run([REFJ])
    assert ON_GPU in r.stderr, r.stderr[-300:]
    assert "continuing on the CPU" not in r.stderr, r.stderr[-300:]
    assert r.returncode == 0 and "greedy match: 20/20" in r.stdout, r.stdout[-300:]


@pytest.mark.gpu
def test_engine_greedy_gate_batched_prompt_on_gpu():
    """The 8-token prompt as one batched step (each GDN layer one chunked
    omh_gdn_prefill, each attention layer one 8-token omh_attn_forward),
    then 20 greedy decode steps: 20/20."""
    r = run([REFJ], OMH_BATCH_PROMPT="1")
    assert ON_GPU in r.stderr and "continuing on the CPU" not in r.stderr, r.stderr[-300:]
    assert r.returncode == 0 and "greedy match: 20/20" in r.stdout, r.stdout[-300:]


@pytest.mark.gpu
def test_engine_teacher_forced_gate_on_gpu():
    """All 28 positions of full_ids in one batched step on the GPU against
    tf_argmax: 28/28."""
    r = run(["--tf", REFJ])
    assert ON_GPU in r.stderr and "continuing on the CPU" not in r.stderr, r.stderr[-300:]
    assert r.returncode == 0 and "teacher-forced match: 28/28" in r.stdout, r.stdout[-300:]


# ---- serve mode (PROTOCOL.md: JSON lines on stdin/stdout; qwen.c:566-607) ----

def _ref_ids():
    with open(REFJ) as f:
        r = json.load(f)
    return r["prompt_ids"], r["full_ids"]


def serve(**env):
    """Three requests through `qwen_hip --serve`: the prompt from position 0
    (reset:true), a warm continuation of the same conversation (reset:false:
    the ids are appended after the 8 + 20 tokens already consumed), then the
    prompt again from zero (reset:true).  Returns {id: [generated ids]}."""
    prompt, _ = _ref_ids()
    reqs = [{"id": 1, "ids": prompt, "n": 20, "reset": True},
            {"id": 2, "ids": [7, 7, 3, 100, 5], "n": 6, "reset": False},
            {"id": 3, "ids": prompt, "n": 20, "reset": True}]
    r = run(["--serve"], stdin="".join(json.dumps(q) + "\n" for q in reqs), **env)
    assert r.returncode == 0, r.stderr[-300:]
    out, done = {}, set()
    lines = [json.loads(ln) for ln in r.stdout.splitlines() if ln.strip()]
    assert lines and lines[0].get("ready") is True, r.stdout[:200]
    for m in lines[1:]:
        assert "error" not in m, m
        if "tok" in m:
            out.setdefault(m["id"], []).append(m["tok"])
        elif m.get("done"):
            assert m["n_out"] == len(out.get(m["id"], [])), m
            done.add(m["id"])
    assert done == {1, 2, 3}, r.stdout[-300:]
    return out, r


def test_engine_serve_cpu_batched_prompt_equals_token_loop():
    """OM_HIP=0: the hooked serve loop's batched prompt (default) gives the
    reference's greedy continuation for a fresh prompt, carries the state on
    reset:false exactly as the reference's token-by-token loop
    (OMH_BATCH_PROMPT=0) does, and restarts from zero on reset:true."""
    _, full = _ref_ids()
    batched, _ = serve(OM_HIP="0")
    loop, _ = serve(OM_HIP="0", OMH_BATCH_PROMPT="0")
    assert batched == loop
    assert batched[1] == full[8:28]
    assert batched[3] == batched[1]


@pytest.mark.gpu
def test_engine_serve_on_gpu():
    """`qwen_hip --serve` with the GDN and attention layers on the GPU: each
    request's ids are one batched prompt step (chunked omh_gdn_prefill per GDN
    layer), reset:true zeroes the device states (omh_gdn_state_reset),
    reset:false continues from them.  Every generated id equals the CPU
    engine's (OM_HIP=0, the reference's token-by-token loop), and the fresh
    prompt gives full_ids."""
    _, full = _ref_ids()
    gpu, r = serve()
    assert ON_GPU in r.stderr and "continuing on the CPU" not in r.stderr, r.stderr[-300:]
    cpu, _ = serve(OM_HIP="0", OMH_BATCH_PROMPT="0")
    assert gpu == cpu
    assert gpu[1] == full[8:28] and gpu[3] == gpu[1]


@pytest.mark.gpu
@pytest.mark.parametrize("layer,batched", [(4, "1"), (7, "0")])
def test_engine_fallback_mid_step_hands_state_back(layer, batched):
    """A GPU call that fails mid-step (forced from the host through the
    hooks' OMH_TEST_FAIL_LAYER, no GPU fault): every layer already on the GPU
    hands its state back (GDN state, attention cache rows up to the step's
    last token) and the engine finishes on the CPU with the reference's
    greedy 20/20.  Layer 4 fails inside the batched prompt step, after
    attention layer 3 wrote all 8 prompt rows on the device; layer 7 (an
    attention layer) fails in the first token-by-token step."""
    r = run([REFJ], OMH_BATCH_PROMPT=batched, OMH_TEST_FAIL_LAYER=str(layer))
    assert ON_GPU in r.stderr and "injected by OMH_TEST_FAIL_LAYER" in r.stderr, r.stderr[-300:]
    assert r.returncode == 0 and "greedy match: 20/20" in r.stdout, r.stdout[-300:]


# ---- the engine's int8 container (stream mode, qwen.c:213-218, 269-274) ----

@pytest.fixture(scope="module")
def int8_container(tmp_path_factory):
    """The reference tiny model rewritten as an int8 container
    (tests/golden/make_int8_container.py: routed experts as row-wise int8 +
    .qs scales, the reference converter's layout).  Loading it puts the
    engine in stream mode: it quantises the GDN in_proj_qkv / in_proj_z /
    out_proj and the attention projections to int8 twins at load, so the
    hooks upload those twins (the m->stream branches of omh_gdn_upload and
    omh_attn_upload)."""
    from tests.golden.make_int8_container import write_container
    dst = str(tmp_path_factory.mktemp("qwen_tiny_i8"))
    write_container(TINY, dst)
    return dst


STREAM = "streaming experts: int8 container"


def test_engine_int8_container_cpu_gates(int8_container):
    """OM_HIP=0 on the int8 container: the engine runs in stream mode and
    still reproduces the reference's greedy 20/20 and teacher-forced 28/28."""
    r = run([REFJ], OM_HIP="0", SNAP=int8_container)
    assert STREAM in r.stderr and r.returncode == 0 and "greedy match: 20/20" in r.stdout, r.stdout[-300:]
    r = run(["--tf", REFJ], OM_HIP="0", SNAP=int8_container)
    assert r.returncode == 0 and "teacher-forced match: 28/28" in r.stdout, r.stdout[-300:]


def _engine_line(out):
    return [ln for ln in out.splitlines() if ln.startswith("engine   :")][0]


@pytest.mark.gpu
@pytest.mark.parametrize("args,env", [([REFJ], {}), ([REFJ], {"OMH_BATCH_PROMPT": "1"}), (["--tf", REFJ], {})],
                         ids=["greedy", "greedy-batched-prompt", "teacher-forced"])
def test_engine_int8_container_on_gpu(int8_container, args, env):
    """Stream mode with the GDN and attention layers on the GPU as int8
    twins (in_proj / out_proj and q/k/v/o through the int8 kernels): the
    same ids as the CPU engine on the same container, and the reference's
    gates (greedy 20/20, teacher-forced 28/28)."""
    gpu = run(args, SNAP=int8_container, **env)
    cpu = run(args, SNAP=int8_container, OM_HIP="0", **env)
    assert STREAM in gpu.stderr and ON_GPU in gpu.stderr, gpu.stderr[-300:]
    assert "continuing on the CPU" not in gpu.stderr, gpu.stderr[-300:]
    assert _engine_line(gpu.stdout) == _engine_line(cpu.stdout)
    assert gpu.returncode == 0, gpu.stdout[-300:]
