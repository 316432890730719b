"""Independent pins of the oracle's sampled tree walk, its penalized row
selection and its sparse-draft residual (oracle/jf_oracle.c: jfo_accept_tree,
jfo_select_row's penalties, draft_q).

Each check states the expected result from the reference's own rules,
written here without the oracle's code:
  - the sampled tree walk (tree.metal:42-58): hand-built trees whose answers
    are worked out by hand, chosen so that a wrong uniform slot, a wrong row
    index for p or q, or a missing chain-child exclusion changes the answer;
    and a chain-shaped sampled tree against the chain acceptance
    (sampling.metal:1399-1423), which the tree must reduce to;
  - penalties (sampling.metal:928-993; Sampling.cpp:50-80): the penalized
    logits of a verify row computed vectorized from a history (prompt bits,
    output counts) and the lane's verify input rows as the reference's
    `drafted` bitmask (row r counts input rows 1..r), then the kept set and
    the greedy token by brute force from those logits;
  - the residual draw with a sparse 16-candidate draft that lists a token
    twice (sampling.metal:700-708: only the first entry counts): the
    speculative-sampling identity, checked to fail when the later entry's
    probability is used instead.
"""
import math

import numpy as np
import pytest

import oracle as O
from test_oracle import FLT_MAX, definitional_kept, pack

NO = O.NO_TOKEN


# ---- sampled tree walk (tree.metal:20-84) ------------------------------------

def _tree(parent, token, chain_rows, chain_q, p, u, tgt, remaining=8, stop=(NO, NO),
          sampled=True):
    tt, ret, acc, path = O.accept_tree(parent, token, chain_rows, chain_q, remaining,
                                       sampled, tgt, target_draft_prob=p, uniforms40=u,
                                       stop=stop)
    return list(tt[:ret]), ret, acc, list(path)


def _uniforms(acceptance, tree_draws=0.99):
    """40 uniforms: slots 8.. from `acceptance`, the tree-draw slots 24..39 set
    to `tree_draws` and every other slot to 0.5, so that reading a wrong slot
    changes the accept/reject decision."""
    u = np.full(40, 0.5, np.float32)
    u[24:40] = tree_draws
    u[8:8 + len(acceptance)] = acceptance
    return u


def test_sampled_tree_accepts_along_the_chain():
    # Chain rows 0-1-2-3 (chain_rows 4), an off-chain branch 0-4-5.
    parent = [0, 0, 1, 2, 0, 4]
    token = [100, 11, 12, 13, 21, 22]
    q = [0.5] * 8
    p = [0.3] * 16  # accept iff u * 0.5 < 0.3, i.e. u < 0.6
    tgt = [7, 8, 9, 10, 21, 22]
    # u[8..10] accept; a walk reading the tree-draw slots (0.99) would reject.
    out, ret, acc, path = _tree(parent, token, 4, q, p, _uniforms([0.1, 0.1, 0.1]), tgt)
    assert path == [0, 1, 2, 3, 3, 3, 3, 3]
    assert out == [11, 12, 13, 10] and acc == 3 and ret == 4


def test_sampled_tree_rejects_then_follows_an_off_chain_child():
    parent = [0, 0, 1, 2, 0, 4]
    token = [100, 11, 12, 13, 21, 22]
    q = [0.5] * 8
    p = [0.3] * 16
    tgt = [21, 8, 9, 10, 22, 99]  # row 0's draw is row 4's token, row 4's row 5's
    # u[8] = 0.9 rejects; slot 24 (tree draw of row 0) = 0.0 would accept.
    out, ret, acc, path = _tree(parent, token, 4, q, p, _uniforms([0.9], tree_draws=0.0), tgt)
    assert path == [0, 4, 5, 5, 5, 5, 5, 5]
    assert out == [21, 22, 99] and acc == 2 and ret == 3


def test_sampled_tree_excludes_the_chain_child_after_a_rejection():
    # Row 0's children: row 1 (the chain) and row 3, both holding token 11.
    parent = [0, 0, 1, 0]
    token = [100, 11, 12, 11]
    q = [0.5] * 8
    p = [0.3] * 16
    tgt = [11, 12, 40, 55]
    u = _uniforms([0.9, 0.0])  # reject at row 0; row 1 would accept at once
    out, ret, acc, path = _tree(parent, token, 3, q, p, u, tgt)
    assert path[:2] == [0, 3]
    assert out == [11, 55] and acc == 1 and ret == 2
    # A greedy lane takes the lowest matching child, the chain's row 1, and
    # then row 1's child row 2 (its target token 12 is row 2's token).
    out, ret, acc, path = _tree(parent, token, 3, q, p, u, tgt, sampled=False)
    assert path[:3] == [0, 1, 2]
    assert out == [11, 12, 40] and acc == 2


def test_sampled_tree_past_the_chain_end_matches_every_child():
    # chain_rows 2: rows 0-1 are the chain; row 2 (a child of row 1) is not,
    # so after the chain's last row the walk may take row 2 by its token.
    parent = [0, 0, 1, 2]
    token = [100, 11, 12, 13]
    q = [0.5] * 8
    p = [0.3] * 16
    tgt = [5, 12, 13, 77]
    out, ret, acc, path = _tree(parent, token, 2, q, p, _uniforms([0.1]), tgt)
    assert path == [0, 1, 2, 3, 3, 3, 3, 3]
    assert out == [11, 12, 13, 77] and acc == 3


def test_sampled_tree_reads_p_and_q_of_the_current_row():
    parent = [0, 0, 1, 2]
    token = [100, 11, 12, 13]
    u = _uniforms([0.1, 0.1, 0.1])
    tgt = [5, 6, 7, 8]
    # Row 0 accepts (0.1 * 0.5 < 0.3); row 1 rejects (0.1 * 0.5 < 0.01 fails).
    # With p or q read one row later, row 0 would reject.
    p = [0.3, 0.01, 0.3, 0.3]
    q = [0.5, 0.5, 0.5]
    out, ret, acc, path = _tree(parent, token, 4, q, p, u, tgt)
    assert path[:2] == [0, 1] and out == [11, 6] and acc == 1
    q = [0.5, 5.0, 0.5]  # now q of row 1 decides: 0.1 * 5 < 0.3 fails
    p = [0.3, 0.3, 0.3, 0.3]
    out, ret, acc, path = _tree(parent, token, 4, q, p, u, tgt)
    assert path[:2] == [0, 1] and out == [11, 6] and acc == 1


def test_sampled_tree_depth_cap_and_stop_cut():
    n = 12
    parent = [0] + list(range(n - 1))
    token = [100] + [10 + r for r in range(1, n)]
    q = [0.5] * 8
    p = [0.9] * 16
    tgt = list(range(200, 200 + n))
    u = _uniforms([0.1] * 7)
    out, ret, acc, path = _tree(parent, token, n, q, p, u, tgt)
    assert path == list(range(8))  # JUSTFIT_TREE_MAXIMUM_DEPTH rows
    assert out == [11, 12, 13, 14, 15, 16, 17, 207] and acc == 7 and ret == 8
    out, ret, acc, _ = _tree(parent, token, n, q, p, u, tgt, remaining=5)
    assert ret == 5 and acc == 7
    out, ret, acc, _ = _tree(parent, token, n, q, p, u, tgt, stop=(13, NO))
    assert out == [11, 12, 13] and ret == 3 and acc == 7


def test_chain_shaped_sampled_tree_equals_the_sampled_chain():
    rng = np.random.default_rng(31)
    for trial in range(400):
        n = int(rng.integers(2, 9))  # rows, <= 8 (the tree's depth cap)
        drafts = rng.integers(0, 6, n - 1).astype(np.uint32)
        parent = [0] + list(range(n - 1))
        token = [int(rng.integers(0, 6))] + [int(d) for d in drafts]
        q = rng.uniform(0.05, 1.0, n - 1).astype(np.float32)
        p = rng.uniform(0.0, 1.0, 16).astype(np.float32)
        u = rng.random(40).astype(np.float32)
        tgt = rng.integers(0, 6, n).astype(np.uint32)
        remaining = int(rng.integers(1, n + 1))
        stop = (int(rng.integers(0, 8)), NO)
        t_out, t_ret, t_acc, _ = _tree(parent, token, n, list(q), p, u, tgt,
                                       remaining=remaining, stop=stop)
        # The chain lists each draft token among 16 candidates at q.
        ids = np.full((n - 1, 16), NO, np.uint32)
        probs = np.zeros((n - 1, 16), np.float32)
        for i in range(n - 1):
            slot = int(rng.integers(0, 16))
            ids[i] = np.arange(1000, 1016)
            probs[i] = rng.random(16).astype(np.float32)
            ids[i, slot] = drafts[i]
            probs[i, slot] = q[i]
        c_out, c_ret, c_acc = O.accept_chain(n - 1, remaining, True, drafts, tgt,
                                             ids, probs, p, u, stop=stop)
        assert (t_acc, t_ret) == (c_acc, c_ret), trial
        assert t_out == list(c_out[:c_ret]), trial


# ---- penalized selection (sampling.metal:928-993) ---------------------------

def penalized_logits(x, history, generated, mark_prompt, inputs, verify_row, pol):
    """The logits of verify row `verify_row` after decode_sample_penalize_verify,
    vectorized: the table word of every token (Sampling.cpp:50-71: bit 31 for a
    prompt token when marked, plus the count of generated tokens), the lane's
    verify input rows as a per-token `drafted` bitmask, row r counting bits
    1..r, then penalize_logit with the saturating clamp."""
    V = x.size
    h = np.asarray(history, np.int64)
    prompt, gen = h[:len(h) - generated], h[len(h) - generated:]
    counts = np.bincount(gen, minlength=V).astype(np.int64)
    in_prompt = np.zeros(V, bool)
    if mark_prompt:
        in_prompt[prompt] = True
    drafted = np.zeros(V, np.int64)
    for row in range(1, len(inputs)):
        drafted[inputs[row]] |= 1 << row
    within = drafted & ((2 << verify_row) - 2)
    count = counts + np.array([bin(int(b)).count("1") for b in within])
    active = pol.repetition != 1.0 or pol.presence != 0.0 or pol.frequency != 0.0
    touched = (count > 0) | in_prompt
    if not active:
        return x.copy()
    rep = np.float32(pol.repetition)
    inv = min(np.float32(1.0) / rep, FLT_MAX)
    with np.errstate(over="ignore", invalid="ignore"):
        v = x * np.where(x > 0, inv, rep).astype(np.float32)
        low = (np.float32(pol.frequency) * count.astype(np.float32)) + np.float32(pol.presence)
        v = np.where(count > 0, v - low.astype(np.float32), v).astype(np.float32)
    v = np.where(np.isnan(v), -FLT_MAX, np.clip(v, -FLT_MAX, FLT_MAX)).astype(np.float32)
    return np.where(touched, v, x).astype(np.float32)


def _oracle_words(V, history, generated, mark_prompt):
    rc, words = O.rebuild_penalty_words(V, history, generated, mark_prompt=mark_prompt)
    assert rc == 0
    return words


def penalized_cases(seed, n):
    rng = np.random.default_rng(seed)
    for i in range(n):
        V = int(rng.integers(4, 40))
        x = np.round(rng.normal(0, 2, V), int(rng.integers(0, 3))).astype(np.float32)
        if i % 4 == 0:
            x[rng.integers(0, V)] = np.nan  # penalized NaN -> -FLT_MAX
        if i % 6 == 0:
            x[rng.integers(0, V)] = -np.inf
        if i % 9 == 0:
            x[rng.integers(0, V)] = np.float32(3e38)  # saturates under penalties
        H = int(rng.integers(1, 3 * V))
        history = rng.integers(0, min(V, 12), H)  # low ids: repeats
        generated = int(rng.integers(0, H))
        mark = bool(rng.integers(0, 2))
        inputs = rng.integers(0, min(V, 12), 8)
        verify_row = int(rng.integers(0, 8))
        adm = rng.random(V) < 0.85
        adm[rng.integers(0, V)] = True
        pol = O.policy(top_k=int(rng.integers(0, V + 2)),
                       temperature=float(rng.choice([0.0, 0.5, 1.0, 1.3])),
                       top_p=float(rng.choice([1.0, 0.6, 0.9])),
                       min_p=float(rng.choice([0.0, 0.1])),
                       repetition=float(rng.choice([1.0, 1.3, 0.7, 2.0])),
                       presence=float(rng.choice([0.0, 0.5, -1.5, 2.0])),
                       frequency=float(rng.choice([0.0, 0.3, -0.7, 2.0])),
                       constrained=True)
        yield V, x, history, generated, mark, inputs, verify_row, adm, pol


def test_penalized_kept_sets_and_greedy_by_brute_force():
    checked_nan = checked_prompt_only = 0
    for case in penalized_cases(41, 400):
        V, x, history, generated, mark, inputs, r, adm, pol = case
        xp = penalized_logits(x, history, generated, mark, inputs, r, pol)
        words = _oracle_words(V, history, generated, mark)
        extra = np.asarray(inputs[1:r + 1], np.uint32)
        if pol.temperature == 0.0:
            tok = O.select_row(V, pol, logits=x, mask=pack(adm), words=words,
                               extra=extra if extra.size else None)[0]
            ok = adm & ~np.isnan(xp)
            if not ok.any():
                want = O.NO_TOKEN
            else:
                y = np.where(ok, xp, -np.inf)
                want = int(np.argmax(y))  # first maximum: the lowest id
                if y[want] == -np.inf:
                    want = int(np.flatnonzero(ok)[0])
            assert tok == want, case
        else:
            want, wq = definitional_kept(xp, adm, pol)
            tok, _, _, _, ids, _ = O.select_row(V, pol, logits=x, mask=pack(adm), words=words,
                                                extra=extra if extra.size else None,
                                                uniform=0.37, kept_capacity=64)
            assert list(ids) == want, case
        nan_pen = np.isnan(x) & (xp == -FLT_MAX)
        checked_nan += int(nan_pen.any())
        checked_prompt_only += int(mark and pol.repetition != 1.0)
    assert checked_nan > 10 and checked_prompt_only > 50


def test_penalties_touch_the_kept_set():
    """The composition is exercised: on these cases the penalized kept set
    differs from the unpenalized one, so a dropped penalty term fails above."""
    differs = 0
    for case in penalized_cases(41, 400):
        V, x, history, generated, mark, inputs, r, adm, pol = case
        if pol.temperature == 0.0:
            continue
        xp = penalized_logits(x, history, generated, mark, inputs, r, pol)
        a, _ = definitional_kept(xp, adm, pol)
        b, _ = definitional_kept(x, adm, pol)
        # Nor may the verify extras be dropped.
        c, _ = definitional_kept(penalized_logits(x, history, generated, mark, inputs[:1], 0, pol),
                                 adm, pol)
        differs += (a != b) + (a != c)
    assert differs > 100


# ---- sparse-draft residual (sampling.metal:694-829, 700-708) ----------------

def _emitted(V, x, pol, ids, probs, q_of):
    """The emitted distribution of one speculative step: the draft proposes d
    with probability q_of[d], the target accepts it when u q < p(d), and a
    rejection draws from the oracle's residual (uniforms on a grid)."""
    _, _, _, _, kid, kpr = O.select_row(V, pol, logits=x, kept_capacity=V)
    target = np.zeros(V)
    target[kid] = kpr
    grid = 1 << 11
    emitted = np.zeros(V)
    for d in range(V):
        if q_of[d] <= 0:
            continue
        res = np.zeros(V)
        pd = None
        for k in range(grid):
            u = float(np.float32(k / grid))
            t, pdk, *_ = O.select_row(V, pol, logits=x, uniform=u, draft_token=d,
                                      cand_ids=ids, cand_probs=probs)
            res[t] += 1.0 / grid
            pd = pdk
        assert abs(pd - target[d]) <= 1e-6
        acc = min(1.0, target[d] / q_of[d])
        emitted += q_of[d] * (acc * np.eye(V)[d] + (1 - acc) * res)
    return emitted, target


def test_sparse_draft_residual_with_a_duplicated_candidate():
    rng = np.random.default_rng(12)
    V = 10
    x = rng.normal(0, 1.0, V).astype(np.float32)
    pol = O.policy(temperature=1.0)
    # Five distinct candidates with q summing to 1; token `dup` listed again
    # later with another probability; the rest of the 16 slots empty.
    toks = [1, 4, 6, 7, 9]
    q = rng.dirichlet(np.ones(5)).astype(np.float32)
    _, _, _, _, kid, kpr = O.select_row(V, pol, logits=x, kept_capacity=V)
    p_of = dict(zip(kid.tolist(), kpr.tolist()))
    # The duplicate is a token the target favours more than the draft (so its
    # residual is positive), listed again with a probability above p.
    dup = max(toks, key=lambda t: p_of[t] - q[toks.index(t)])
    assert p_of[dup] > q[toks.index(dup)]
    ids = np.full(16, NO, np.uint32)
    probs = np.zeros(16, np.float32)
    ids[:5], probs[:5] = toks, q
    ids[9], probs[9] = dup, np.float32(min(1.0, p_of[dup] + 0.3))
    probs[12] = 0.77  # an empty slot's probability is never read
    q_of = np.zeros(V)
    q_of[toks] = q
    emitted, target = _emitted(V, x, pol, ids, probs, q_of)
    np.testing.assert_allclose(emitted, target, atol=3e-3)
    # Sensitivity: with the later entry's probability first (the lookup a
    # last-match would make), the residual and the identity both change.
    ids2, probs2 = ids.copy(), probs.copy()
    k = toks.index(dup)
    probs2[k], probs2[9] = probs[9], probs[k]
    wrong, _ = _emitted(V, x, pol, ids2, probs2, q_of)
    assert np.abs(wrong - target).max() > 1e-2
