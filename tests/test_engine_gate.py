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
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ENGINE = os.path.join(ROOT, "tests", "engine", "_build", "qwen_hip")
TINY = os.path.join(ROOT, "tests", "golden", "qwen_tiny")
REFJ = os.path.join(TINY, "ref_qwen.json")
ON_GPU = "om_hip: GDN and attention layers on the GPU"


def run(args, **env):
    if not os.path.exists(ENGINE):
        pytest.fail(f"{ENGINE} is not built: run __graft_entry__.build() where the reference sources are present")
    e = dict(os.environ, SNAP=TINY)
    e.pop("OM_HIP", None)
    e.pop("OMH_BATCH_PROMPT", None)
    e.update(env)
    r = subprocess.run([ENGINE] + args, env=e, capture_output=True, text=True, timeout=300)
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
