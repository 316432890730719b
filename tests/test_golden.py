"""The committed fixtures of tests/golden (seeded inputs and the oracle's
outputs, written by tests/golden/make_golden.py): the oracle must still give
them (CPU), and the HIP library must give them bit for bit (GPU)."""
import json
import os

import numpy as np
import pytest

import jf_sampler as J
from harness import assert_same, run_gpu, run_oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
META = json.load(open(os.path.join(HERE, "select_cases.json")))
DATA = np.load(os.path.join(HERE, "select_cases.npz"), allow_pickle=False)


def case_inputs(m):
    name = m["name"]
    kw = {k.split("/")[2]: DATA[k] for k in DATA.files if k.startswith(f"{name}/in/")}
    if m.get("histories") is not None:
        kw["histories"] = [None if h is None else np.array(h, np.uint32) for h in m["histories"]]
        kw["generated"] = m["generated"]
        kw["mark_prompt"] = m["mark_prompt"]
    for k in ("kept_capacity", "drafted_rows"):
        if m.get(k) is not None:
            kw[k] = m[k]
    if m.get("stop"):
        kw["stop"] = tuple(m["stop"])
    want = {k.split("/")[2]: DATA[k] for k in DATA.files if k.startswith(f"{name}/out/")}
    return [J.policy(**p) for p in m["policies"]], kw, want


@pytest.mark.parametrize("m", META, ids=[m["name"] for m in META])
def test_oracle_reproduces_fixture(m):
    pols, kw, want = case_inputs(m)
    got = run_oracle(m["V"], pols, **kw)
    assert_same(got, want)
    for k in ("kept_probs",):
        if k in want:
            np.testing.assert_array_equal(got[k], want[k])


@pytest.mark.gpu
@pytest.mark.parametrize("m", META, ids=[m["name"] for m in META])
def test_gpu_reproduces_fixture(m):
    pols, kw, want = case_inputs(m)
    print(f"golden case {m['name']}", flush=True)
    got = run_gpu(m["V"], pols, **kw)
    assert_same(got, want)
