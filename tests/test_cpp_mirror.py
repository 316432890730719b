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


# ---- the widest verify step (sampling_mirror verify16) ------------------------

V16, ROWS16, LANES16 = 248320, 16, 4


def logits16():
    r = np.arange(LANES16 * ROWS16, dtype=np.uint64)[:, None]
    t = np.arange(V16, dtype=np.uint64)[None, :]
    return (((t * 48271 + r * 16807) % 10007) / 1000.0 - 5.0).astype(np.float32)


def inputs16():
    i = np.arange(LANES16 * ROWS16, dtype=np.uint64)
    return ((i * 7717 + 3) % V16).astype(np.uint32)


def candidates16():
    inp = inputs16()
    c = np.zeros((LANES16, ROWS16 - 1, 16), np.uint32)
    p = np.full((LANES16, ROWS16 - 1, 16), 0.01, np.float32)
    for l in range(LANES16):
        for r in range(ROWS16 - 1):
            for j in range(16):
                c[l, r, j] = inp[l * ROWS16 + r + 1] if j == 0 else (r * 5303 + j * 9721 + l) % V16
            p[l, r, 0] = 0.6
    return c, p


def history16(t):
    inp = inputs16()
    h = ((np.arange(1500, dtype=np.uint64) * 131071 + t * 977) % V16).astype(np.uint32)
    lane = 0 if t == 1 else 2
    for i in range(40):
        h[1000 + i] = inp[lane * ROWS16 + 1 + (i % 5)]
    return h


@pytest.mark.gpu
def test_mirror_verify_4_lanes_16_rows_one_call():
    """addVerify over 4 lanes x 16 rows at V = 248,320 in one selection call
    (per-row mask, draft, candidate and extra-token addressing), with two
    penalized lanes counting their verify inputs, sparse drafts, the
    correction uniform and the tree uniforms; then addAcceptance. Bit-exact
    against the oracle row by row (Sampling.cpp:149-172, 278-328)."""
    got = run("verify16")
    assert got["gpu_failures"] == 0
    x = logits16()
    inp = inputs16()
    cand, cprob = candidates16()
    words = {0: O.rebuild_penalty_words(V16, history16(1), 700, None, True)[1],
             2: O.rebuild_penalty_words(V16, history16(3), 700, None, True)[1]}
    pols = [O.policy(temperature=0.9, top_k=40, top_p=0.92, repetition=1.15, presence=0.4,
                     frequency=0.25),
            O.policy(temperature=0.7, top_k=20), None, O.policy()]
    pols[2] = pols[0]
    for tree, key in ((False, "verify"), (True, "tree")):
        drafted_rows = 7 if tree else ROWS16 - 1
        vt = np.zeros(LANES16 * ROWS16, np.uint32)
        vp = np.zeros(LANES16 * ROWS16, np.float32)
        for l in range(LANES16):
            u = uniforms(l)
            for r in range(ROWS16):
                g = l * ROWS16 + r
                drafted = r < drafted_rows
                t, dp = O.select_row(
                    V16, pols[l], logits=x[g], words=words.get(l),
                    extra=inp[l * ROWS16 + 1:l * ROWS16 + 1 + r] if l in words else None,
                    uniform=float(u[24 + r] if tree else u[15]),
                    draft_token=int(inp[g + 1]) if drafted else NO,
                    cand_ids=cand[l, r] if drafted else None,
                    cand_probs=cprob[l, r] if drafted else None)[:2]
                vt[g], vp[g] = t, dp
        np.testing.assert_array_equal(np.array(got[f"{key}_tokens"], np.uint32), vt, err_msg=key)
        np.testing.assert_array_equal(np.array(got[f"{key}_probs_bits"], np.uint32),
                                      vp.view(np.uint32), err_msg=key)
        if tree:
            continue
        for l, remaining in enumerate([16, 9, 12, 16]):
            sl = slice(l * ROWS16, (l + 1) * ROWS16)
            tt, ret, acc = O.accept_chain(
                ROWS16 - 1, remaining, pols[l].temperature > 0, inp[l * ROWS16 + 1:(l + 1) * ROWS16],
                vt[sl], cand_ids=cand[l], cand_probs=cprob[l], target_draft_prob=vp[sl],
                uniforms40=uniforms(l))
            np.testing.assert_array_equal(np.array(got["accepted_tokens"][sl], np.uint32), tt)
            assert got["retained"][l] == ret and got["accepted"][l] == acc, (l, ret, acc)
