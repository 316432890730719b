"""Pins of the CPU oracle (oracle/jf_oracle.c) against closed forms, published
known answers, brute force and statistics. The reference ships no fixtures for
this path (its C++ tests are not shipped), so each function of the oracle is
checked here against an independent formulation; the HIP build is then held
bit-exact to the oracle in tests/test_gpu_*.py."""
import ctypes
import math
import struct
from fractions import Fraction

import numpy as np
import pytest

import oracle as O

FLT_MAX = np.float32(3.4028234663852886e38)
_libm = ctypes.CDLL("libm.so.6")
_libm.logf.argtypes = [ctypes.c_float]
_libm.logf.restype = ctypes.c_float
LOGF = _libm.logf


def f32(x):
    return np.float32(x)


def bits(x):
    return struct.unpack("<I", struct.pack("<f", float(x)))[0]


# ---- order ---------------------------------------------------------------

def test_logit_key_is_the_float_order():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.normal(0, 10, 2000).astype(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, FLT_MAX, -FLT_MAX, 1e-45, -1e-45],
                 dtype=np.float32)])
    keys = [O.lib().jfo_logit_key(float(v)) for v in vals]
    for i in range(0, len(vals), 7):
        for j in range(0, len(vals), 13):
            a, b = vals[i], vals[j]
            assert (keys[i] > keys[j]) == (a > b)
            assert (keys[i] == keys[j]) == (a == b)
    assert O.lib().jfo_logit_key(0.0) == O.lib().jfo_logit_key(-0.0)
    assert O.lib().jfo_logit_key(float("-inf")) == 0x007FFFFF
    for v in vals:
        back = O.lib().jfo_key_logit(O.lib().jfo_logit_key(float(v)))
        assert bits(back) == (0 if v == 0 else bits(v))


# ---- exp -------------------------------------------------------------------

def ulp_distance(a, b):
    ia = np.int64(np.float32(a).view(np.int32))
    ib = np.int64(np.float32(b).view(np.int32))
    return abs(int(ia) - int(ib))


def test_expf_against_double_exp():
    worst = 0
    for x in np.linspace(-86.0, 0.0, 40001, dtype=np.float32):
        got = O.lib().jfo_expf(float(x))
        ref = np.float32(math.exp(float(x)))
        worst = max(worst, ulp_distance(got, ref))
    assert worst <= 2, worst
    assert O.lib().jfo_expf(0.0) == 1.0
    assert O.lib().jfo_expf(-86.5) == 0.0
    assert O.lib().jfo_expf(float("-inf")) == 0.0
    # monotone non-decreasing over a dense sweep
    xs = np.linspace(-30.0, 0.0, 100001, dtype=np.float32)
    ys = [O.lib().jfo_expf(float(x)) for x in xs]
    assert all(ys[i] <= ys[i + 1] for i in range(len(ys) - 1))


def test_floor_mul_is_exact():
    rng = np.random.default_rng(1)
    for _ in range(5000):
        a = int(rng.integers(0, 1 << 62))
        f = np.float32(rng.random())
        if rng.random() < 0.1:
            f = np.float32(rng.random() * 1e-30)
        want = math.floor(a * Fraction(float(f)))
        assert O.lib().jfo_floor_mul(a, float(f)) == want
    assert O.lib().jfo_floor_mul(12345, 1.0) == 12345
    assert O.lib().jfo_floor_mul(12345, 0.0) == 0
    assert O.lib().jfo_floor_mul(12345, float("nan")) == 0


def f32_of_int(n):
    """n rounded to the nearest float32 (ties to even), by integer
    arithmetic: numpy's int -> float32 passes through float64 and can round
    twice."""
    e = n.bit_length() - 24
    if e <= 0:
        return np.float32(n)
    q, r = divmod(n, 1 << e)
    half = 1 << (e - 1)
    if r > half or (r == half and q & 1):
        q += 1
    return np.float32(float(q << e))


def residual_reference(w, mass, q):
    """max(w - floor(q * m), 0) for m the mass as a float32 and the product
    rounded to float32; q NaN or <= 0 takes nothing off, a product at or
    above 2^44 leaves nothing."""
    q = np.float32(q)
    if not q > 0:
        return w
    x = q * f32_of_int(mass)  # float32 product, ties to even
    if not x < np.float32(2.0 ** 44):
        return 0
    return max(w - math.floor(Fraction(float(x))), 0)


def test_residual_weight():
    """jfo_residual, the drafted rows' residual weight, against float32
    products and exact integers; the edges: q NaN/negative/zero/infinite,
    q >= 1, products on both sides of 2^32 (the kernels' two-word split) and
    of 2^44 (nothing left), and masses whose float rounds up or down."""
    L = O.lib()
    rng = np.random.default_rng(7)
    cases = []
    for _ in range(4000):
        mass = int(rng.integers(1 << 44, 1 << 63))
        w = int(rng.integers(0, (1 << 44) + 1))
        kind = rng.integers(0, 4)
        if kind == 0:
            q = rng.random()
        elif kind == 1:
            q = rng.random() * 1e-6
        elif kind == 2:
            # products near 2^32 and 2^44
            target = 2.0 ** (32 if rng.random() < 0.5 else 44)
            q = target / float(f32_of_int(mass)) * (1 + (rng.random() - 0.5) * 1e-6)
        else:
            q = rng.random() * 1e-30
        cases.append((w, mass, float(np.float32(q))))
    cases += [(5, 1 << 44, float("nan")), (5, 1 << 44, -0.5), (5, 1 << 44, 0.0),
              (5, 1 << 44, float("inf")), (1 << 44, 1 << 44, 1.0), (1 << 44, (1 << 45) - 1, 1.0),
              (1 << 44, (1 << 44) + 1, 1.0), (123, (1 << 63) - 1, 2.0),
              ((1 << 44) - 1, (1 << 60) + (1 << 36) + 1, 2.0 ** -20)]
    hits32 = 0
    for w, mass, q in cases:
        want = residual_reference(w, mass, q)
        assert L.jfo_residual(w, mass, q) == want, (w, mass, q)
        x = np.float32(q) * f32_of_int(mass) if q > 0 else 0
        hits32 += 2.0 ** 32 <= x < 2.0 ** 44
    assert hits32 > 100
    # Closed forms: no draft mass takes nothing off; q = 1 removes the whole
    # weight (the mass is at least the weight).
    assert L.jfo_residual(777, 1 << 50, 0.0) == 777
    assert L.jfo_residual(1 << 44, 1 << 44, 1.0) == 0


# ---- uniforms -------------------------------------------------------------

def splitmix_reference(state):
    """Vigna's published splitmix64 step: (next state, output)."""
    m = (1 << 64) - 1
    state = (state + 0x9E3779B97F4A7C15) & m
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return state, z ^ (z >> 31)


def test_splitmix64_known_answers():
    # Published: splitmix64 seeded with 0 first returns 0xe220a8397b1dcdaf.
    assert O.lib().jfo_splitmix64(0, 1) == 0xE220A8397B1DCDAF
    for seed in (0, 1, 0xDEADBEEF, (1 << 64) - 1):
        state = seed
        for ctr in range(1, 50):
            state, out = splitmix_reference(state)
            assert O.lib().jfo_splitmix64(seed, ctr) == out
            u, c = O.next_uniform(seed, ctr - 1)
            assert c == ctr
            assert u == np.float32((out >> 40) * 2.0 ** -24)


@pytest.mark.parametrize("rows,tree,end", [(8, False, 16), (16, False, 24), (16, True, 40), (8, True, 16)])
def test_stage_cycle_slots(rows, tree, end):
    u, c = O.stage_cycle(77, 5, rows, tree)
    assert c == 5 + end - 1
    assert u[0] == 0 and np.all(u[end:] == 0)
    ctr = 5
    for slot in range(1, end):
        v, ctr = O.next_uniform(77, ctr)
        assert u[slot] == v


# ---- penalties ------------------------------------------------------------

def words_by_dict(V, history, generated, pending, mark_prompt):
    """Sampling.cpp:50-71 restated with dictionaries."""
    prompt = history[:len(history) - generated]
    out = {}
    if mark_prompt:
        for t in prompt:
            out[int(t)] = out.get(int(t), 0) | 0x80000000
    for t in list(history[len(prompt):]) + ([pending] if pending is not None else []):
        out[int(t)] = out.get(int(t), 0) + 1
    dense = np.zeros(V, dtype=np.uint32)
    for t, w in out.items():
        dense[t] = w
    return dense


@pytest.mark.parametrize("mark", [False, True])
def test_penalty_words_rebuild(mark):
    rng = np.random.default_rng(2)
    V = 5000
    for gen in (0, 10, 299):
        h = rng.integers(0, V, 300)
        h[:5] = 7
        rc, words = O.rebuild_penalty_words(V, h, gen, pending=11, mark_prompt=mark)
        assert rc == 0
        np.testing.assert_array_equal(words, words_by_dict(V, h, gen, 11, mark))
    assert O.rebuild_penalty_words(V, [1, 2, 3], 3)[0] == -1
    assert O.rebuild_penalty_words(V, [1, V, 3], 0)[0] == -2
    assert O.rebuild_penalty_words(V, [1, 2, 3], 0, pending=V)[0] == -2


def test_penalize_logit_closed_form():
    L = O.lib()
    rng = np.random.default_rng(3)
    for _ in range(2000):
        v = f32(rng.normal(0, 5))
        c = int(rng.integers(0, 5))
        rep = f32(rng.uniform(0.5, 2))
        inv = L.jfo_repetition_inverse(float(rep))
        pres, freq = f32(rng.uniform(-2, 2)), f32(rng.uniform(-2, 2))
        want = v * (np.float32(inv) if v > 0 else rep)
        if c:
            want = want - (freq * np.float32(c) + pres)
        want = np.clip(want, -FLT_MAX, FLT_MAX)
        got = L.jfo_penalize_logit(float(v), c, float(rep), inv, float(pres), float(freq))
        assert bits(got) == bits(want)
    assert L.jfo_penalize_logit(float("nan"), 1, 1.1, 1 / 1.1, 0.5, 0.3) == -FLT_MAX
    assert L.jfo_penalize_logit(float("inf"), 0, 1.0, 1.0, 0, 0) == FLT_MAX
    assert L.jfo_repetition_inverse(1e-45) == FLT_MAX


# ---- greedy -----------------------------------------------------------------

def test_greedy_matches_argmax_with_lowest_id_ties():
    rng = np.random.default_rng(4)
    V = 3000
    for trial in range(40):
        x = np.round(rng.normal(0, 2, V), 1).astype(np.float32)  # many ties
        allowed = rng.random(V) < 0.3
        mask = pack(allowed)
        stop = (int(rng.integers(0, V)), int(rng.integers(0, V)))
        excl = bool(trial % 2)
        tok = O.select_row(V, O.policy(constrained=True, exclude_stop=excl), logits=x,
                           mask=mask, stop=stop)[0]
        adm = allowed.copy()
        if excl:
            adm[list(stop)] = False
        y = np.where(adm, x, -np.inf)
        want = int(np.argmax(y)) if adm.any() else O.NO_TOKEN
        if adm.any() and y[want] == -np.inf:
            want = int(np.flatnonzero(adm)[0])
        assert tok == want


def test_greedy_sentinels():
    V = 100
    x = np.full(V, np.nan, dtype=np.float32)
    assert O.select_row(V, O.policy(), logits=x)[0] == O.NO_TOKEN
    x = np.full(V, -np.inf, dtype=np.float32)
    assert O.select_row(V, O.policy(), logits=x)[0] == 0
    x[37] = np.nan
    x[50] = 1.0
    assert O.select_row(V, O.policy(), logits=x)[0] == 50
    mask = np.zeros(4, dtype=np.uint32)
    assert O.select_row(V, O.policy(constrained=True), logits=x, mask=mask)[0] == O.NO_TOKEN


def pack(allowed):
    V = allowed.size
    W = (V + 31) // 32
    out = np.zeros(W, dtype=np.uint32)
    for t in np.flatnonzero(allowed):
        out[t // 32] |= np.uint32(1 << (t % 32))
    return out


# ---- sampled: brute force -------------------------------------------------

def definitional_kept(x, adm, p):
    """The kept set by definition: order by pairwise comparison, top-k by
    counting predecessors, min-p by value, top-p by exact prefix masses."""
    L = O.lib()
    V = x.size
    T = np.float32(p.temperature)
    inv_t = np.float32(1.0) / T
    cand = [t for t in range(V) if adm[t] and not np.isnan(x[t])]
    if not cand:
        return [], None
    M = max(np.float32(-FLT_MAX), max(x[t] for t in cand))

    def before(a, b):  # a strictly before b in (logit desc, id asc)
        return x[a] > x[b] or (x[a] == x[b] and a < b)

    if p.min_p > 0:
        # min(M + T log(min_p), M) with the platform's logf, in fp32
        offset = np.float32(T * np.float32(LOGF(np.float32(p.min_p))))
        floor_v = min(np.float32(M + offset), M)
        cand = [t for t in cand if x[t] >= floor_v]
    k = p.top_k if (p.top_k and p.top_k < V) else V
    rank = {t: sum(before(o, t) for o in cand) for t in cand}
    cand = [t for t in cand if rank[t] < k]
    wq = {t: int(np.float32(L.jfo_expf(float(np.float32((x[t] - M) * inv_t)))) * np.float32(2.0 ** 44))
          for t in cand}
    if p.top_p < 1:
        ordered = sorted(cand, key=lambda t: sum(before(o, t) for o in cand))
        mass = sum(wq.values())
        nucleus = math.floor(mass * Fraction(float(np.float32(p.top_p))))
        run = 0
        for i, t in enumerate(ordered):
            run += wq[t]
            if run > nucleus:
                cand = ordered[:i + 1]
                break
    return sorted(cand), wq


def tiny_cases(seed, n):
    rng = np.random.default_rng(seed)
    for i in range(n):
        V = int(rng.integers(4, 48))
        x = np.round(rng.normal(0, 2, V), int(rng.integers(0, 3))).astype(np.float32)
        if i % 5 == 0:
            x[rng.integers(0, V)] = -np.inf
        if i % 7 == 0:
            x[rng.integers(0, V)] = np.nan
        adm = rng.random(V) < 0.8
        adm[rng.integers(0, V)] = True
        p = O.policy(top_k=int(rng.integers(0, V + 2)),
                     temperature=float(rng.choice([0.3, 0.7, 1.0, 1.7])),
                     top_p=float(rng.choice([1.0, 0.5, 0.9, 0.2])),
                     min_p=float(rng.choice([0.0, 0.0, 0.05, 0.3])),
                     constrained=True)
        yield V, x, adm, p


def test_kept_set_brute_force():
    for V, x, adm, p in tiny_cases(5, 300):
        want, wq = definitional_kept(x, adm, p)
        tok, dp, n, M, ids, probs = O.select_row(V, p, logits=x, mask=pack(adm),
                                                 uniform=0.5, kept_capacity=64)
        assert list(ids) == want
        if want and sum(wq[t] for t in want):
            # probabilities against float64 softmax over the kept set
            M64 = max(float(x[t]) for t in want)
            e = np.array([math.exp((float(x[t]) - M64) / float(np.float32(p.temperature))) for t in want])
            ref = e / e.sum()
            big = ref > 1e-30
            np.testing.assert_allclose(probs[big], ref[big], rtol=1e-5, atol=0)
            assert tok in want


def inverse_cdf_counts(weights, grid_bits=16):
    """For u on a 2^grid_bits grid, how often the inverse CDF over integer
    weights (first index whose running sum exceeds floor(u * total)) picks
    each index."""
    total = sum(weights)
    cum = np.cumsum(weights)
    counts = np.zeros(len(weights), dtype=np.int64)
    for k in range(1 << grid_bits):
        target = (k * total) >> grid_bits
        counts[int(np.searchsorted(cum, target, side="right"))] += 1
    return counts


def test_draw_is_the_inverse_cdf():
    rng = np.random.default_rng(6)
    for _ in range(6):
        V = 12
        x = rng.normal(0, 1.5, V).astype(np.float32)
        p = O.policy(temperature=1.0)
        want_ids, wq = definitional_kept(x, np.ones(V, bool), p)
        weights = [wq[t] for t in want_ids]
        want = inverse_cdf_counts(weights, 12)
        got = np.zeros(V, dtype=np.int64)
        for k in range(1 << 12):
            u = float(np.float32(k / 4096.0))
            got[O.select_row(V, p, logits=x, uniform=u)[0]] += 1
        np.testing.assert_array_equal(got[want_ids], want)


def test_residual_restores_the_target_distribution():
    """Speculative sampling: draft d ~ q, accept if u q_d < p_d, else draw
    from the residual; the emitted token is distributed as p."""
    rng = np.random.default_rng(7)
    V = 10
    for trial in range(4):
        x = rng.normal(0, 1.0, V).astype(np.float32)
        q = rng.dirichlet(np.ones(V)).astype(np.float32)
        p = O.policy(temperature=1.0, top_k=[0, 6][trial % 2])
        _, _, _, _, ids, probs = O.select_row(V, p, logits=x, uniform=0.0, kept_capacity=V)
        target = np.zeros(V)
        target[ids] = probs
        emitted = np.zeros(V)
        grid = 1 << 12
        for d in range(V):
            res = np.zeros(V)
            for k in range(grid):
                u = float(np.float32(k / grid))
                t, pd, *_ = O.select_row(V, p, logits=x, uniform=u, draft_token=d, dense_q=q)
                res[t] += 1.0 / grid
            pd = target[d]
            acc = min(1.0, pd / q[d]) if q[d] > 0 else 1.0
            emitted += q[d] * (acc * np.eye(V)[d] + (1 - acc) * res)
        np.testing.assert_allclose(emitted, target, atol=3e-3)


def test_draft_probability_is_kept_weight_over_mass():
    rng = np.random.default_rng(8)
    V = 30
    x = rng.normal(0, 2, V).astype(np.float32)
    p = O.policy(temperature=0.8, top_k=10)
    _, _, _, _, ids, probs = O.select_row(V, p, logits=x, kept_capacity=V)
    for d in range(V):
        dp = O.select_row(V, p, logits=x, draft_token=d,
                          cand_ids=np.array([d] + [O.NO_TOKEN] * 15),
                          cand_probs=np.array([0.01] + [0] * 15))[1]
        want = probs[list(ids).index(d)] if d in ids else 0.0
        assert dp == want


def test_sampled_sentinels():
    V = 64
    p = O.policy(temperature=1.0)
    assert O.select_row(V, p, logits=np.full(V, np.nan, np.float32))[0] == O.NO_TOKEN
    assert O.select_row(V, p, logits=np.full(V, -np.inf, np.float32))[0] == O.NO_TOKEN
    x = np.zeros(V, np.float32)
    x[3] = np.inf
    assert O.select_row(V, p, logits=x)[0] == O.NO_TOKEN


# ---- acceptance -------------------------------------------------------------

def test_chain_greedy_prefix_and_stop():
    tt, ret, acc = O.accept_chain(7, 8, False, [5, 6, 7, 9, 9, 9, 9], [5, 6, 7, 8, 1, 2, 3, 4])
    assert acc == 3 and ret == 4
    tt, ret, acc = O.accept_chain(7, 2, False, [5, 6, 7, 9, 9, 9, 9], [5, 6, 7, 8, 1, 2, 3, 4])
    assert acc == 3 and ret == 2
    tt, ret, acc = O.accept_chain(7, 8, False, [5, 6, 7, 9, 9, 9, 9], [5, 6, 7, 8, 1, 2, 3, 4], stop=(6, O.NO_TOKEN))
    assert acc == 3 and ret == 2


def test_chain_sampled_test():
    ids = np.full((7, 16), O.NO_TOKEN, dtype=np.uint32)
    probs = np.zeros((7, 16), dtype=np.float32)
    draft = [10, 11, 12, 13, 14, 15, 16]
    for i, d in enumerate(draft):
        ids[i, 0], probs[i, 0] = d, 0.5
    u = np.zeros(40, np.float32)
    u[8:15] = [0.1, 0.1, 0.9, 0.1, 0.1, 0.1, 0.1]
    p = np.full(8, 0.2, np.float32)  # accept iff u * 0.5 < 0.2 <=> u < 0.4
    tt, ret, acc = O.accept_chain(7, 8, True, draft, [1, 2, 3, 4, 5, 6, 7, 8], ids, probs, p, u)
    assert acc == 2 and ret == 3
    assert list(tt[:3]) == [10, 11, 3]


def test_tree_chain_shape_equals_chain():
    rng = np.random.default_rng(9)
    for _ in range(50):
        tgt = rng.integers(0, 5, 8)
        toks = [0] + list(rng.integers(0, 5, 7))
        parent = [0] + list(range(7))
        tt, ret, acc, path = O.accept_tree(parent, toks, 0, None, 8, False, tgt)
        ct, cret, cacc = O.accept_chain(7, 8, False, toks[1:], tgt)
        assert acc == cacc and ret == cret
        assert list(tt[:ret]) == list(ct[:ret])


def test_tree_branch_walk():
    parent = [0, 0, 1, 0, 3, 3]
    token = [0, 5, 6, 7, 8, 9]
    # target after row 0 wants 7 (row 3), after row 3 wants 9 (row 5), after row 5 wants 42
    tgt = [7, 0, 0, 9, 0, 42]
    tt, ret, acc, path = O.accept_tree(parent, token, 0, None, 8, False, tgt)
    assert acc == 2 and ret == 3
    assert list(tt[:3]) == [7, 9, 42]
    assert list(path) == [0, 3, 5, 5, 5, 5, 5, 5]


# ---- draft selector (sampling.metal:995-1359) ------------------------------

def _bf16(x):
    """Round-to-nearest-even bf16 bit patterns of float32 values."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16f(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def _top16_lexsort(row):
    """Top 16 by (value desc, id asc) among non-NaN, padded (-inf, NO)."""
    ids = np.arange(len(row))
    ok = ~np.isnan(row)
    v, i = row[ok], ids[ok]
    order = np.lexsort((i, -v.astype(np.float64)))[:16]
    out_ids = np.full(16, O.NO_TOKEN, np.uint32)
    out_v = np.full(16, -np.inf, np.float32)
    out_ids[:len(order)] = i[order]
    out_v[:len(order)] = v[order]
    return out_ids, out_v


@pytest.mark.parametrize("case", ["random", "ties", "neg_inf", "nan", "zeros", "short"])
def test_draft_top16_matches_lexsort(case):
    rng = np.random.default_rng(hash(case) % 1000)
    V = 37 if case == "short" else 20011
    row = rng.normal(0, 2, V).astype(np.float32)
    if case == "ties":
        row = np.round(row, 0).astype(np.float32)
    elif case == "neg_inf":
        row[:] = -np.inf
        row[[3, 77, 900]] = [1.0, -2.0, 5.0]
    elif case == "nan":
        row[::2] = np.nan
        row[1::4] = 9.0
    elif case == "zeros":
        row[:] = -5.0
        row[::3] = 0.0
        row[1::3] = -0.0
    elif case == "short":
        row[5:] = np.nan
    ids, vals = O.draft_top16(row)
    want_ids, want_v = _top16_lexsort(row)
    assert np.array_equal(ids, want_ids)
    assert np.array_equal(vals.view(np.uint32), want_v.view(np.uint32))


def test_draft_edge_against_float64():
    rng = np.random.default_rng(5)
    for _ in range(50):
        pc, h, sc = (_bf16(rng.normal(0, s, 256)) for s in (0.5, 2.0, 0.3))
        got = O.draft_edge(pc, h, sc)
        terms = _bf16f(pc).astype(np.float64) * _bf16f(h) * _bf16f(sc)
        want = terms.sum()
        assert abs(got - want) <= 1e-6 * np.abs(terms).sum() + 1e-30
        # The roles are pinned: the same check fails without the hidden
        # factor or with the codebooks swapped against another hidden row.
        h2 = _bf16(rng.normal(0, 2.0, 256))
        other = (_bf16f(pc).astype(np.float64) * _bf16f(h2) * _bf16f(sc)).sum()
        assert abs(O.draft_edge(pc, h2, sc) - other) <= 1e-6 * np.abs(terms).sum() * 10 + 1e-30
        assert abs(got - (_bf16f(pc).astype(np.float64) * _bf16f(sc)).sum()) > 1e-3


def _draft_inputs(rng, lanes, V):
    logits = rng.normal(0, 2, (lanes * 8, V)).astype(np.float32)
    hidden = _bf16(rng.normal(0, 1, (lanes * 8, 256)))
    pc = _bf16(rng.normal(0, 0.2, (V, 256)))
    sc = _bf16(rng.normal(0, 0.2, (V, 256)))
    anchors = rng.integers(0, V, lanes).astype(np.uint32)
    u = rng.random((lanes, 40)).astype(np.float32)
    return logits, hidden, pc, sc, anchors, u


def test_draft_walk_greedy_and_sampled():
    rng = np.random.default_rng(8)
    lanes, V = 3, 3000
    logits, hidden, pc, sc, anchors, u = _draft_inputs(rng, lanes, V)
    temps = [0.0, 0.8, 1.5]
    sampled = [False, True, True]
    cand, unary, tokens, q = O.draft_select(logits, hidden, pc, sc, anchors, temps, sampled, u)
    for l in range(lanes):
        pred = 0
        for p in range(7):
            ids, vals = _top16_lexsort(logits[l * 8 + p + 1])
            assert np.array_equal(cand[l, p], ids) and np.array_equal(unary[l, p], vals)
            prev = [int(anchors[l])] if p == 0 else [int(x) for x in cand[l, p - 1]]
            pid = min(prev[pred], V - 1)
            edges = np.array([O.draft_edge(pc[pid], hidden[l * 8 + p + 1], sc[min(int(c), V - 1)])
                              for c in cand[l, p]], np.float32)
            scores = unary[l, p] + edges
            if not sampled[l]:
                sel = int(np.argmax(scores))  # first of equal maxima
                assert np.all(q[l, p] == 0)
            else:
                z = (scores.astype(np.float64) - scores.max()) / temps[l]
                want = np.exp(z) / np.exp(z).sum()
                assert np.allclose(q[l, p], want, rtol=1e-5, atol=1e-7)
                cum = np.cumsum(q[l, p], dtype=np.float32)  # sequential fp32
                hit = np.nonzero(cum > u[l, 1 + p])[0]
                sel = int(hit[0]) if len(hit) else 15
            assert tokens[l, p] == cand[l, p, sel]
            pred = sel


# ---- tree gather (tree.metal:86-107) ---------------------------------------

from gather_cases import gather_case, gather_closed_form

@pytest.mark.parametrize("shape", [dict(), dict(columns=48, inner=8, inner_stride=2, outer_stride=20),
                                   dict(columns=30, inner=5, inner_stride=1, outer_stride=7)])
def test_tree_gather_closed_form(shape):
    rng = np.random.default_rng(len(shape))
    data, path, retained, p = gather_case(rng, **shape)
    got = O.tree_gather(data, path, retained, **p)
    assert np.array_equal(got, gather_closed_form(data, path, retained, p))
