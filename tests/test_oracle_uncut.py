"""Pins of the oracle's arithmetic for sampled rows with no min-p, top-k or
top-p cut, whose exact mass is kept per 8192-token chunk against the chunk's
own maximum and rescaled to the row maximum once per chunk (jf_oracle.c,
uncut_select; the rescale r_c = exp((m_c - M) / T) in double, carried as a
32-bit significand R_c and a shift s_c). Rows span several chunks; few tokens
are admitted, so the checks enumerate them:
  - jfo_exp64 against the C library's exp (double) over [-708, 0] and its
    edges; the packed rescale against exp of the same float arguments (R in
    [2^31, 2^32), relative error at most 2^-32 at any offset); jfo_scale_by
    against Python's exact integers;
  - every chunk holding the row maximum (every rescale exactly 1): the draw
    equals the row-maximum inverse CDF over quantized weights, bit for bit;
  - chunk maxima from 0 down to -80 T below the row maximum, at T = 0.7, 1
    and 2: every reported probability against float64 softmax at 1e-5
    relative, and equal (1e-5) to the same token's probability on the cut
    path (a masked row with top_k = V - 1 keeps the same set);
  - the draw's inverse CDF in id order: each kept token's interval of the
    2^24 uniforms, found by bisection, is its float64 softmax probability
    within two uniform steps;
  - the speculative-sampling identity for drafted rows across chunks, and the
    plain draw when no residual mass remains;
  - p(draft) equal to the draft's reported kept probability;
  - tokens on both sides of the chunk boundaries (multiples of 8192), far
    below the row maximum, at their softmax probability;
  - rows of -inf only: the sentinel, with every token kept at probability 0."""
import math

import numpy as np

import oracle as O
from test_oracle import inverse_cdf_counts, pack

CHUNK = 8192


def structured_row(rng, V, per_chunk, chunk_offsets, T):
    """Logits with `per_chunk` admitted tokens in each chunk, chunk c's
    values shifted by chunk_offsets[c] (None: nothing admitted there)."""
    x = rng.normal(0, 1.0, V).astype(np.float32)
    adm = np.zeros(V, bool)
    for c, off in enumerate(chunk_offsets):
        lo, hi = c * CHUNK, min((c + 1) * CHUNK, V)
        if off is None or lo >= V:
            continue
        ids = rng.choice(np.arange(lo, hi), size=min(per_chunk, hi - lo), replace=False)
        adm[ids] = True
        x[ids] = (x[ids] * np.float32(1.5) + np.float32(off)).astype(np.float32)
    return x, adm


def far_row(rng, T, offsets):
    """Chunk c's maximum at offsets[c] * T below 3.0 (the row maximum in
    chunk 0), five more admitted tokens up to 2 T below it, plus a partial
    last chunk; unadmitted tokens hold N(0, 1) values."""
    V = len(offsets) * CHUNK + 333
    Tf = np.float32(T)
    x = rng.normal(0, 1.0, V).astype(np.float32)
    adm = np.zeros(V, bool)
    for c, d in enumerate(offsets):
        ids = rng.choice(np.arange(c * CHUNK, (c + 1) * CHUNK), 6, replace=False)
        adm[ids] = True
        top = np.float32(np.float32(3.0) - np.float32(d) * Tf)
        x[ids] = (top - Tf * (rng.random(6).astype(np.float32) * np.float32(2))).astype(np.float32)
        x[ids[0]] = top
    adm[V - 5] = True
    x[V - 5] = np.float32(3.0 - 3 * T)
    return V, x, adm


def softmax_of(x, adm, T):
    ids = np.flatnonzero(adm & ~np.isnan(x))
    v = x[ids].astype(np.float64)
    M = v.max()
    e = np.exp((v - M) / float(np.float32(T)))
    return ids, e / e.sum()


def draws(V, p, x, adm, grid, **kw):
    out = np.empty(grid, np.int64)
    for k in range(grid):
        u = float(np.float32(k / grid))
        out[k] = O.select_row(V, p, logits=x, mask=pack(adm), uniform=u, **kw)[0]
    return out


def test_exp64_against_the_c_library():
    L = O.lib()
    rng = np.random.default_rng(30)
    xs = np.concatenate([-rng.random(20000) * 708.0, -rng.random(20000) * 2.0,
                         [0.0, -0.0, -1e-300, -0.3465735902799726, -0.34657359028,
                          -707.999, -708.0, -1.5, -86.0, -745.0 / 2]])
    for x in xs:
        got, want = L.jfo_exp64(float(x)), math.exp(float(x))
        assert abs(got - want) <= 2 * math.ulp(want), (x, got, want)
    assert L.jfo_exp64(0.0) == 1.0 and L.jfo_exp64(-0.0) == 1.0
    assert L.jfo_exp64(-708.0001) == 0.0 and L.jfo_exp64(float("-inf")) == 0.0
    assert L.jfo_exp64(float("nan")) == 0.0


def test_chunk_scale_is_a_32_bit_significand_and_a_shift():
    L = O.lib()
    rng = np.random.default_rng(36)
    for T in (0.7, 1.0, 2.0):
        inv_t = np.float32(1.0) / np.float32(T)
        for d in np.concatenate([-rng.random(3000) * 500.0, -rng.random(3000) * 30.0]):
            m = np.float32(d)
            sc = L.jfo_chunk_scale(float(m), 0.0, float(inv_t))
            R, s = sc & 0xFFFFFFFF, sc >> 32
            want = math.exp(float(m) * float(inv_t))
            if want < 1e-300:
                continue
            assert 2 ** 31 <= R < 2 ** 32
            assert abs(R * 2.0 ** -s - want) <= (2.0 ** -32 + 4 * 2.0 ** -52) * want
    # The row maximum's own chunk: exactly 1. Underflow: R = 0, s = 64.
    assert L.jfo_chunk_scale(5.0, 5.0, 1.0) == (31 << 32) | (1 << 31)
    assert L.jfo_chunk_scale(-1e30, 0.0, 1.0) == 64 << 32
    for _ in range(2000):
        x = int(rng.integers(0, 2 ** 63, dtype=np.uint64))
        R = int(rng.integers(2 ** 31, 2 ** 32))
        s = int(rng.integers(31, 140))
        assert L.jfo_scale_by(x, (s << 32) | R) == (x * R) >> s
    assert L.jfo_scale_by(2 ** 63 - 1, 64 << 32) == 0


def test_equal_chunk_maxima_give_the_row_maximum_draw():
    rng = np.random.default_rng(31)
    V = 3 * CHUNK + 77
    for T in (0.6, 1.0, 1.7):
        x, adm = structured_row(rng, V, 6, [0.0, 0.5, -0.4, 0.2], T)
        ids = np.flatnonzero(adm)
        M = np.float32(x[ids].max())
        for c in range(4):  # each chunk holds the row maximum
            x[ids[(ids >= c * CHUNK) & (ids < (c + 1) * CHUNK)][0]] = M
        p = O.policy(temperature=T, constrained=True)
        inv_t = np.float32(1.0) / np.float32(T)
        L = O.lib()
        wq = [int(np.float32(L.jfo_expf(float(np.float32((x[t] - M) * inv_t)))) *
                  np.float32(2.0 ** 44)) for t in ids]
        want = inverse_cdf_counts(wq, 12)
        got = draws(V, p, x, adm, 1 << 12)
        np.testing.assert_array_equal([np.sum(got == t) for t in ids], want)


OFFSETS = [0, 5, 10, 15, 20, 22, 30, 45, 60, 80]


def test_far_chunks_match_softmax_and_the_cut_path():
    """Chunk maxima down to 80 T below the row maximum (tokens to 82 T): the
    probabilities that the reference computes as w / sum with
    w = exp((x - M) / T) (sampling.metal:38-40, 647-652, 828-829), within
    1e-5 relative of float64 softmax, and of the cut path's own."""
    rng = np.random.default_rng(37)
    for T in (0.7, 1.0, 2.0):
        for _ in range(2):
            V, x, adm = far_row(rng, T, OFFSETS)
            ids, ref = softmax_of(x, adm, T)
            assert ref.min() > 1e-37  # every token a normal float
            p = O.policy(temperature=T, constrained=True)
            _, _, n, _, kid, kpr = O.select_row(V, p, logits=x, mask=pack(adm),
                                                kept_capacity=128)
            assert n == len(ids) and list(kid) == list(ids)
            np.testing.assert_allclose(kpr, ref, rtol=1e-5, atol=0)
            # top_k = V - 1 on a masked row keeps the same set by the cut path.
            pc = O.policy(temperature=T, constrained=True, top_k=V - 1)
            _, _, n2, _, kid2, kpr2 = O.select_row(V, pc, logits=x, mask=pack(adm),
                                                   kept_capacity=128)
            assert list(kid2) == list(ids)
            np.testing.assert_allclose(kpr, kpr2, rtol=1e-5, atol=0)
            # p(draft) of tokens in the far chunks.
            for t in ids[::7]:
                dp = O.select_row(V, p, logits=x, mask=pack(adm), draft_token=int(t),
                                  cand_ids=np.array([t] + [O.NO_TOKEN] * 15),
                                  cand_probs=np.array([0.5] + [0] * 15))[1]
                assert dp == kpr[list(ids).index(t)]


def cdf_intervals(V, p, x, adm, ids):
    """Each kept token's share of the 2^24 uniforms u = k 2^-24 (the draw is
    monotone in u, in id order), by bisection on the first k that draws a
    later token."""
    def draw(k):
        return O.select_row(V, p, logits=x, mask=pack(adm), uniform=k * 2.0 ** -24)[0]
    starts = []
    for t in ids[1:]:
        lo, hi = 0, 1 << 24  # draw(hi) >= t is taken as true at hi = 2^24
        while lo < hi:
            mid = (lo + hi) // 2
            if draw(mid) >= t:
                hi = mid
            else:
                lo = mid + 1
        starts.append(lo)
    edges = np.array([0] + starts + [1 << 24], dtype=np.float64)
    return np.diff(edges) * 2.0 ** -24


def test_draw_intervals_are_the_softmax_probabilities():
    rng = np.random.default_rng(38)
    V = 5 * CHUNK + 1234
    for T, offs in ((1.0, [0.0, -1.3, None, -7.0, -2.0, -0.5]),
                    (0.7, [-3.0, 0.0, -0.2, -12.0, 1.0, -4.0]),
                    (2.0, [None, 0.0, -5.0, -0.01, None, -30.0])):
        x, adm = structured_row(rng, V, 5, offs, T)
        p = O.policy(temperature=T, constrained=True)
        ids, ref = softmax_of(x, adm, T)
        got = cdf_intervals(V, p, x, adm, ids)
        assert np.all(np.abs(got - ref) <= 2 * 2.0 ** -24), np.abs(got - ref).max()


def test_residual_restores_the_target_distribution_across_chunks():
    rng = np.random.default_rng(33)
    V = 2 * CHUNK + 100
    x, adm = structured_row(rng, V, 4, [0.0, -0.7, 0.3], 1.0)
    p = O.policy(temperature=1.0, constrained=True)
    ids, _ = softmax_of(x, adm, 1.0)
    _, _, _, _, kid, kpr = O.select_row(V, p, logits=x, mask=pack(adm), kept_capacity=64)
    target = np.zeros(V)
    target[kid] = kpr
    q = np.zeros(V, np.float32)
    q[ids] = rng.dirichlet(np.ones(len(ids))).astype(np.float32) * np.float32(0.9)
    q[5] = np.float32(0.1)  # draft mass on a token the row does not admit
    emitted = np.zeros(V)
    grid = 1 << 10
    for d in list(ids) + [5]:
        res = np.bincount(draws(V, p, x, adm, grid, draft_token=int(d), dense_q=q),
                          minlength=V) / grid
        pd = target[d]
        acc = min(1.0, pd / q[d]) if q[d] > 0 else 1.0
        emitted += q[d] * (acc * np.eye(V)[d] + (1 - acc) * res)
    np.testing.assert_allclose(emitted[ids], target[ids], atol=4e-3)


def test_draft_probability_is_its_kept_probability():
    rng = np.random.default_rng(34)
    V = 3 * CHUNK + 5
    x, adm = structured_row(rng, V, 5, [0.0, -2.5, 0.4, -1.0], 0.8)
    p = O.policy(temperature=0.8, constrained=True)
    _, _, _, _, kid, kpr = O.select_row(V, p, logits=x, mask=pack(adm), kept_capacity=64)
    for d in list(kid) + [7]:
        dp = O.select_row(V, p, logits=x, mask=pack(adm), draft_token=int(d),
                          cand_ids=np.array([d] + [O.NO_TOKEN] * 15),
                          cand_probs=np.array([0.01] + [0] * 15))[1]
        want = kpr[list(kid).index(d)] if d in kid else 0.0
        assert dp == want


def test_drafted_row_without_residual_mass_draws_plainly():
    """q >= p on every token leaves no residual mass: the drafted row draws
    exactly as the undrafted row does (sampling.metal:739-765)."""
    rng = np.random.default_rng(35)
    V = 2 * CHUNK + 31
    x, adm = structured_row(rng, V, 5, [0.0, -1.5, 0.7], 1.0)
    p = O.policy(temperature=1.0, constrained=True)
    q = np.ones(V, np.float32)
    plain = draws(V, p, x, adm, 256)
    drafted = draws(V, p, x, adm, 256, draft_token=int(np.flatnonzero(adm)[0]), dense_q=q)
    np.testing.assert_array_equal(drafted, plain)


def test_chunk_boundaries_keep_far_tokens():
    """Tokens on both sides of token 8192 and of 2 * 8192, 25 T below the row
    maximum, whether or not their chunk holds anything higher, report their
    softmax probability (1e-11 here) at 1e-5 relative."""
    V = 3 * CHUNK + 10
    for T in (1.0, 0.7):
        x = np.full(V, -np.inf, np.float32)
        x[100] = 0.0                                  # the row maximum, chunk 0
        for t in (8000, 8191, 8192, 16383, 16385):    # chunks 0, 0, 1, 1, 2
            x[t] = np.float32(-25.0 * T)
        x[16384] = np.float32(-1.0 * T)               # chunk 2's own maximum
        p = O.policy(temperature=T)
        _, _, n, _, kid, kpr = O.select_row(V, p, logits=x, kept_capacity=V)
        prob = dict(zip(kid.tolist(), kpr.tolist()))
        ids = [100, 8000, 8191, 8192, 16383, 16384, 16385]
        e = {t: math.exp((float(x[t]) - 0.0) / float(np.float32(T))) for t in ids}
        z = sum(e.values())
        for t in ids:
            assert abs(prob[t] - e[t] / z) <= 1e-5 * e[t] / z, (T, t, prob[t], e[t] / z)


def test_minus_infinity_rows_keep_every_token_at_zero():
    V = 2 * CHUNK + 9
    p = O.policy(temperature=1.0)
    tok, dp, n, M, kid, kpr = O.select_row(V, p, logits=np.full(V, -np.inf, np.float32),
                                           kept_capacity=16)
    assert tok == O.NO_TOKEN and n == V
    assert list(kid) == list(range(16)) and np.all(kpr == 0)
    assert math.isfinite(M)
