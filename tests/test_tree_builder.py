"""The draft tree builder (jf_build_draft_tree, the reference's
buildDraftTree, Runtime.cpp:58-174): host code, so these run on the CPU.
Pinned three ways: field-for-field equality with the oracle's independent
Python restatement (heapq frontier), the structural invariants of the
layout (preorder parents, depths, root-to-leaf copies, first-copy
ownership), and the greedy/sampled chain as the leftmost path."""
import numpy as np
import pytest

import jf_sampler as J
import oracle as O


def inputs(seed, V=50000):
    rng = np.random.default_rng(seed)
    cand = rng.integers(0, V, (7, 16)).astype(np.uint32)
    unary = rng.normal(0, 2, (7, 16)).astype(np.float32)
    edges = rng.normal(0, 1, (7, 16, 16)).astype(np.float32)
    return cand, unary, edges, int(rng.integers(0, V))


def check_layout(t, cand, rows):
    n = t["rows"]
    assert n == rows
    assert t["depth"][0] == 0
    for r in range(1, n):
        p = t["parent"][r]
        assert p < r and t["depth"][r] == t["depth"][p] + 1
        assert t["token"][r] in cand[t["depth"][r] - 1]
    owner = {}
    for c in range(t["copies"]):
        path = t["path"][c][:t["path_length"][c]]
        assert path[0] == 0
        for d in range(1, len(path)):
            assert t["parent"][path[d]] == path[d - 1] and t["depth"][path[d]] == d
        for r in path:
            owner.setdefault(r, c)
    assert sorted(owner) == list(range(n))
    for r in range(n):
        assert t["copy"][r] == owner[r]


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("rows", [1, 2, 5, 9, 16])
@pytest.mark.parametrize("chained", [False, True])
def test_tree_builder_matches_oracle(seed, rows, chained):
    cand, unary, edges, anchor = inputs(seed)
    picks = np.random.default_rng(seed + 100).integers(0, 16, 7).astype(np.uint32) if chained else None
    got = J.build_draft_tree(cand, unary, edges, anchor, rows, picks)
    want = O.build_draft_tree(cand, unary, edges, anchor, rows, picks)
    for k in ("rows", "copies", "parent", "depth", "copy", "token", "path_length", "path"):
        assert got[k] == want[k], k
    assert got["expected"] == want["expected"]
    assert got["chain_expected"] == want["chain_expected"]
    check_layout(got, cand, rows)
    assert got["token"][0] == anchor


@pytest.mark.parametrize("seed", range(4))
def test_leftmost_path_is_the_chain(seed):
    cand, unary, edges, anchor = inputs(seed)
    # Greedy: each position's best candidate after the one before (the
    # selector's own walk) is the leftmost path while it lasts.
    t = J.build_draft_tree(cand, unary, edges, anchor, 16)
    pred, row = 0, 0
    for p in range(7):
        best = int(np.argmax(unary[p].astype(np.float64) + edges[p, pred].astype(np.float64)))
        if row + 1 >= t["rows"] or t["parent"][row + 1] != row:
            break
        row += 1
        assert t["token"][row] == cand[p, best]
        pred = best
    assert row >= 1
    # Sampled: the forced chain is rows 1..7 whatever its scores.
    picks = np.array([15, 0, 7, 3, 9, 1, 12], np.uint32)
    t = J.build_draft_tree(cand, unary, edges, anchor, 16, picks)
    for p in range(7):
        assert t["parent"][p + 1] == p and t["token"][p + 1] == cand[p, picks[p]]


def test_tree_builder_rejects_bad_arguments():
    cand, unary, edges, anchor = inputs(0)
    for rows in (0, 17):
        with pytest.raises(J.JfError):
            J.build_draft_tree(cand, unary, edges, anchor, rows)
    with pytest.raises(J.JfError):
        J.build_draft_tree(cand, unary, edges, anchor, 8, np.full(7, 16, np.uint32))
