"""Pins of the oracle's draw for sampled rows with no min-p, top-k or top-p
cut, whose exact mass is kept per 8192-token chunk against the chunk's own
maximum and rescaled to the row maximum once per chunk (jf_oracle.c,
uncut_select). Rows span several chunks; few tokens are admitted, so the
checks enumerate them:
  - every chunk holding the row maximum (every rescale exactly 2^32): the draw
    equals the row-maximum inverse CDF over quantized weights, bit for bit;
  - chunks with different maxima: reported probabilities against float64
    softmax, the draw's frequencies over a uniform grid against the same
    softmax (within the grid step), and the draw monotone in u;
  - the speculative-sampling identity for drafted rows across chunks, and
    the plain draw when no residual mass remains;
  - p(draft) equal to the draft's reported kept probability;
  - the chunk boundaries at multiples of 8192 (a chunk far below the row
    maximum rescales to zero, tokens as low beside the maximum do not);
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


def test_rescaled_chunks_match_softmax():
    rng = np.random.default_rng(32)
    V = 4 * CHUNK + 1234
    # Chunk maxima far apart, a chunk with nothing admitted, a partial last chunk.
    for T, offs in ((1.0, [0.0, -1.3, None, -7.0, -2.0]), (0.7, [-3.0, 0.0, -0.2, -40.0, 1.0]),
                    (2.0, [None, 0.0, -5.0, -0.01, None])):
        x, adm = structured_row(rng, V, 5, offs, T)
        p = O.policy(temperature=T, constrained=True)
        ids, ref = softmax_of(x, adm, T)
        _, _, n, _, kid, kpr = O.select_row(V, p, logits=x, mask=pack(adm), kept_capacity=64)
        assert n == len(ids) and list(kid) == list(ids)
        np.testing.assert_allclose(kpr, ref, rtol=2e-5, atol=1e-9)
        grid = 1 << 13
        got = draws(V, p, x, adm, grid)
        assert np.all(np.diff(got) >= 0)  # the inverse CDF in id order
        freq = np.array([np.sum(got == t) for t in ids]) / grid
        assert np.all(np.abs(freq - ref) <= 1.0 / grid + 1e-5)


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


def test_chunk_boundaries_are_every_8192_tokens():
    """A chunk whose maximum is more than about 22 T below the row maximum
    rescales by floor(e^-22 * 2^32) = 0: its tokens get probability exactly
    0, while tokens as low inside a chunk that holds the maximum keep their
    weight. Both sides of token 8192 and of 2 * 8192 are probed."""
    V = 3 * CHUNK + 10
    T = 1.0
    x = np.full(V, -np.inf, np.float32)
    x[100] = 0.0                      # the row maximum, chunk 0
    x[8000] = -25.0                   # chunk 0 (with the maximum): kept weight
    x[8191] = -25.0
    x[8192] = -25.0                   # chunk 1 (nothing higher): rescaled to 0
    x[16383] = -25.0
    x[16384] = -1.0                   # chunk 2: its own maximum, weight e^-1
    x[16385] = -25.0                  # same chunk as -1: e^-25 kept
    p = O.policy(temperature=T)
    _, _, n, _, kid, kpr = O.select_row(V, p, logits=x, kept_capacity=V)
    prob = dict(zip(kid.tolist(), kpr.tolist()))
    e = {t: math.exp(float(x[t])) for t in (100, 8000, 8191, 16384, 16385)}
    z = sum(e.values())
    for t in (8000, 8191, 16385):
        assert prob[t] > 0 and abs(prob[t] - e[t] / z) <= 1e-3 * e[t] / z
    assert prob[8192] == 0.0 and prob[16383] == 0.0
    assert abs(prob[16384] - e[16384] / z) <= 1e-6


def test_minus_infinity_rows_keep_every_token_at_zero():
    V = 2 * CHUNK + 9
    p = O.policy(temperature=1.0)
    tok, dp, n, M, kid, kpr = O.select_row(V, p, logits=np.full(V, -np.inf, np.float32),
                                           kept_capacity=16)
    assert tok == O.NO_TOKEN and n == V
    assert list(kid) == list(range(16)) and np.all(kpr == 0)
    assert math.isfinite(M)
