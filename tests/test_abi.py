"""CPU checks of the C ABI library: it loads, exports every symbol the header
declares, and its host-side helpers agree with the oracle and the reference's
error behaviour. No compute call is made (there is no GPU here)."""
import ctypes
import os
import re

import numpy as np
import pytest

import jf_sampler as J
import oracle as O

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(REPO, "include", "jf_sampler.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]*?\b(jf_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    declared = header_functions()
    assert sorted(J.EXPORTS) == declared
    lib = J.lib()  # loads torch's HIP runtime first: one runtime per process
    for name in declared:
        assert hasattr(lib, name), name


def test_next_uniform_matches_oracle():
    for seed in (0, 3, 2**63 + 5):
        c1 = c2 = 0
        for _ in range(100):
            u1, c1 = J.next_uniform(seed, c1)
            u2, c2 = O.next_uniform(seed, c2)
            assert u1 == u2 and c1 == c2


@pytest.mark.parametrize("rows,tree", [(8, False), (16, False), (16, True)])
def test_stage_cycle_matches_oracle(rows, tree):
    a, ca = J.stage_cycle(99, 4, rows, tree)
    b, cb = O.stage_cycle(99, 4, rows, tree)
    np.testing.assert_array_equal(a, b)
    assert ca == cb


def test_penalty_words_match_oracle_and_errors():
    rng = np.random.default_rng(1)
    V = 4096
    h = rng.integers(0, V, 500).astype(np.uint32)
    for gen, pend, mark in ((0, None, True), (100, 17, False), (499, 3, True)):
        w = np.zeros(V, np.uint32)
        J.rebuild_penalty_words(w, h, gen, pend, mark)
        rc, ref = O.rebuild_penalty_words(V, h, gen, pend, mark)
        np.testing.assert_array_equal(w, ref)
        sel = rng.integers(0, V, 9)
        J.count_penalty_tokens(w, sel)
        for t in sel:
            ref[t] += 1
        np.testing.assert_array_equal(w, ref)
    w = np.zeros(V, np.uint32)
    with pytest.raises(J.JfError) as e:
        J.rebuild_penalty_words(w, [1, 2], 2, None, False)
    assert e.value.code == J.JF_ERR_LOGIC and "no prompt" in e.value.message
    with pytest.raises(J.JfError) as e:
        J.rebuild_penalty_words(w, [1, V], 0, None, False)
    assert e.value.code == J.JF_ERR_INVALID_ARGUMENT and "outside the vocabulary" in e.value.message
    with pytest.raises(J.JfError):
        J.count_penalty_tokens(w, [V + 5])


def test_policy_validation_matches_reference_rules():
    ok = [J.policy(), J.policy(temperature=0.7, top_k=50, top_p=0.9),
          J.policy(temperature=2e-38, min_p=1.0), J.policy(presence=2.0, frequency=-2.0)]
    bad = [J.policy(temperature=1e-39), J.policy(temperature=float("inf")),
           J.policy(top_p=0.0), J.policy(top_p=1.01), J.policy(min_p=-0.1),
           J.policy(min_p=1.5), J.policy(presence=2.5), J.policy(repetition=0.0),
           J.policy(repetition=float("nan")), J.policy(frequency=float("nan"))]
    for p in ok:
        J.validate(p)
        assert O.lib().jfo_policy_valid(ctypes.byref(O.policy_from(p))) == 0
    for p in bad:
        with pytest.raises(J.JfError) as e:
            J.validate(p)
        assert e.value.code == J.JF_ERR_INVALID_ARGUMENT
        assert O.lib().jfo_policy_valid(ctypes.byref(O.policy_from(p))) != 0


def test_sampler_row_count_is_bounded():
    """Rows are rejected before any device call: none and more than 2^22 (the
    fast launch packs its first row in 14 bits of 256-row units)."""
    for rows, msg in ((0, "row count"), ((1 << 22) + 1, "exceeds 4194304")):
        h = ctypes.c_void_p()
        rc = J.lib().jf_sampler_create(1000, rows, ctypes.byref(h))
        assert rc == J.JF_ERR_INVALID_ARGUMENT and not h.value
        assert msg in J.lib().jf_last_error().decode()


def test_product_has_no_oracle_or_fallback():
    """The product never loads the oracle and has no CPU compute path."""
    pkg = os.path.join(REPO, "justfit-llm_amd")
    for root, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".cpp", ".hip", ".h", ".hpp")):
                text = open(os.path.join(root, f)).read()
                assert "jf_oracle" not in text and "import oracle" not in text, f
