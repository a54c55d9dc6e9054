"""End-to-end gate on the reference's tiny model (oracle/qwen_tiny,
ref_qwen.json): greedy 20/20 against `full_ids` (the reference engine's own
validation, qwen.c:621-658) and teacher-forced 28/28 against `tf_argmax`
(transformers' chunked path, make_qwen_oracle.py:68-69).

The non-GDN layers run in the host restatement (tests/qwen_tiny.py).  On
the CPU the GDN layers are the C oracle (this pins the host model and the
oracle at token level); on the GPU they are libom_hip.so, one token per
call (omh_gdn_decode) or the whole sequence in one chunked prefill
(omh_gdn_prefill)."""
import numpy as np
import pytest

from tests import qwen_tiny as q


def _count(got, exp):
    return sum(int(a == b) for a, b in zip(got, exp))


def test_host_model_with_oracle_gdn_greedy_20_of_20():
    m = q.TinyQwen(q.OracleGdn)
    got, exp = q.greedy(m)
    assert len(exp) == 20 and got == exp, f"{_count(got, exp)}/20: {got} vs {exp}"


def test_host_model_with_oracle_gdn_teacher_forced_28_of_28():
    m = q.TinyQwen(q.OracleGdn)
    got, exp = q.teacher_forced(m)
    assert len(exp) == 28 and got == exp, f"{_count(got, exp)}/28"


@pytest.mark.gpu
def test_tiny_greedy_with_gpu_gdn_decode():
    m = q.TinyQwen(q.HipGdn, first_li=900)
    try:
        got, exp = q.greedy(m)
    finally:
        m.close()
    assert got == exp, f"greedy {_count(got, exp)}/20: {got} vs {exp}"


@pytest.mark.gpu
def test_tiny_teacher_forced_with_gpu_gdn_prefill():
    """All 28 positions in one forward: each GDN layer is one chunked
    prefill of 28 tokens on the GPU."""
    m = q.TinyQwen(q.HipGdn, first_li=920, batched=True)
    try:
        got, exp = q.teacher_forced(m)
    finally:
        m.close()
    assert got == exp, f"teacher-forced {_count(got, exp)}/28"


@pytest.mark.gpu
def test_tiny_prompt_prefill_then_gpu_decode_matches_oracle_logits():
    """The batched step the reference lacks (its prompt goes token by token,
    qwen.c:637): the 8-token prompt in one chunked prefill, then 20 greedy
    decode steps; tokens 20/20 and logits close to the all-oracle run."""
    ref = q.TinyQwen(q.OracleGdn)
    m = q.TinyQwen(q.HipGdn, first_li=940, batched=True)
    try:
        prompt, full = m.ref["prompt_ids"], m.ref["full_ids"]
        lg = m.forward(prompt)[-1]
        lr = ref.forward(prompt)[-1]
        m.gdn.batched = False
        worst = float(np.abs(lg - lr).max())
        got = []
        for i in range(len(full) - len(prompt)):
            best = int(np.argmax(lg))
            got.append(best)
            if i < len(full) - len(prompt) - 1:
                lg = m.forward([best])[0]
                lr = ref.forward([best])[0]
                worst = max(worst, float(np.abs(lg - lr).max()))
    finally:
        m.close()
    assert got == list(full[len(prompt):]), f"{_count(got, full[len(prompt):])}/20"
    assert worst < 1e-3, f"logits differ from the oracle run by {worst:.3g}"
