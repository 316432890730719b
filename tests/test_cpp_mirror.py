"""The C++ operator mirror justfit::hip::Sampling (justfit-llm_amd/csrc/
sampling.hpp), driven by tests/cpp/sampling_mirror.cpp the way the
reference's Runtime drives ops::Sampling: argument checks and host helpers
on the CPU, and addInitial / addVerify / addAcceptance on the GPU against
the CPU oracle on the same deterministic inputs."""
import json
import os
import subprocess

import numpy as np
import pytest

import jf_sampler as J
import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "_build", "sampling_mirror")
V, ROWS, LANES = 1000, 8, 2
NO = 0xFFFFFFFF


def run(mode):
    assert os.path.exists(BIN), "build first: python tests/cpp/build.py"
    res = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr + res.stdout
    return json.loads(res.stdout)


def test_mirror_checks_and_helpers():
    assert run("cpu")["cpu_failures"] == 0


# The inputs of sampling_mirror.cpp, restated.
def logits():
    r = np.arange(LANES * ROWS, dtype=np.uint64)[:, None]
    t = np.arange(V, dtype=np.uint64)[None, :]
    return (((t * 7919 + r * 104729) % 2003) / 200.0 - 5.0).astype(np.float32)


def uniforms(lane):
    s = np.arange(40, dtype=np.uint64)
    return ((((lane * 40 + s) * 37) % 101) / 101.0).astype(np.float32)


def inputs():
    i = np.arange(LANES * ROWS, dtype=np.uint64)
    return ((i * 131 + 17) % V).astype(np.uint32)


def candidates():
    inp = inputs()
    c = np.zeros((LANES, ROWS - 1, 16), np.uint32)
    p = np.full((LANES, ROWS - 1, 16), 0.02, np.float32)
    for l in range(LANES):
        for r in range(ROWS - 1):
            for j in range(16):
                c[l, r, j] = inp[l * ROWS + r + 1] if j == 0 else (r * 53 + j * 97) % V
            p[l, r, 0] = 0.7
    return c, p


@pytest.mark.gpu
def test_mirror_selection_and_acceptance_on_gpu():
    got = run("gpu")
    assert got["gpu_failures"] == 0
    x = logits()
    inp = inputs()
    cand, cprob = candidates()
    _, w0 = O.rebuild_penalty_words(V, [5, 17, 17, 999], 2, None, True)
    words = [w0, np.zeros(V, np.uint32)]
    # addInitial: lane l selects row l * 8 with uniform slot 0.
    pols = [O.policy(repetition=1.2), O.policy(temperature=0.8, top_k=30, top_p=0.9)]
    for l in range(LANES):
        t = O.select_row(V, pols[l], logits=x[l * ROWS], words=words[l] if l == 0 else None,
                         uniform=float(uniforms(l)[0]))[0]
        assert got["initial_tokens"][l] == t, (l, got["initial_tokens"][l], t)
    # addVerify: every row, draft tokens 1..7, extra tokens 1..r, the
    # correction uniform (slot 15) for every row.
    pv = O.policy(temperature=1.0, top_k=50, presence=0.3)
    vt = np.zeros(LANES * ROWS, np.uint32)
    vp = np.zeros(LANES * ROWS, np.float32)
    for l in range(LANES):
        for r in range(ROWS):
            drafted = r < ROWS - 1
            t, dp = O.select_row(
                V, pv, logits=x[l * ROWS + r], words=words[l],
                extra=inp[l * ROWS + 1:l * ROWS + 1 + r], uniform=float(uniforms(l)[15]),
                draft_token=int(inp[l * ROWS + r + 1]) if drafted else NO,
                cand_ids=cand[l, r] if drafted else None,
                cand_probs=cprob[l, r] if drafted else None)[:2]
            vt[l * ROWS + r], vp[l * ROWS + r] = t, dp
    np.testing.assert_array_equal(np.array(got["verify_tokens"], np.uint32), vt)
    np.testing.assert_array_equal(np.array(got["verify_probs_bits"], np.uint32), vp.view(np.uint32))
    # addAcceptance over the verified rows.
    for l, remaining in enumerate([8, 5]):
        tt, ret, acc = O.accept_chain(
            ROWS - 1, remaining, True, inp[l * ROWS + 1:(l + 1) * ROWS], vt[l * ROWS:(l + 1) * ROWS],
            cand_ids=cand[l], cand_probs=cprob[l], target_draft_prob=vp[l * ROWS:(l + 1) * ROWS],
            uniforms40=uniforms(l))
        np.testing.assert_array_equal(np.array(got["accepted_tokens"][l * ROWS:(l + 1) * ROWS], np.uint32), tt)
        assert got["retained"][l] == ret and got["accepted"][l] == acc, (l, ret, acc)
