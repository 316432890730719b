"""GPU parity of jf_sample (through the C ABI) against the CPU oracle.

Bar: bit-exact tokens, kept sets, kept probabilities and draft probabilities
(the oracle restates the same fp32 weight and exact integer sums); greedy ids
bit-exact. Full-size configs C1-C3 and C5 are compared row by row; edge cases
cover ties, empty/NaN/inf rows, masks, stop exclusion, vocabularies that do
not fill a chunk, the multi-pass stages (top-k disabled with top-p or
min-p, large k), the two-pass draw of rows with no cut (with plain, dense
and sparse drafts, and mixed with cut rows in one launch), and chi-square
tests of 10^6 draws through the merge and through the two-pass draw."""
import numpy as np
import pytest

import jf_sampler as J
from jf_sampler import workloads as WL
from harness import NO, assert_same, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def both(V, policies, **kw):
    print(f"case V={V} rows={len(policies)} keys={sorted(kw)}", flush=True)
    g = run_gpu(V, policies, **kw)
    r = run_oracle(V, policies, **kw)
    return g, r


def test_c1_greedy_repetition():
    c = WL.config1()
    pol = [J.policy(**c["policy"])]
    g, r = both(c["V"], pol, logits=c["logits"], histories=c["histories"],
                generated=c["generated"], mark_prompt=[True])
    assert_same(g, r, check_draft=False)


def test_c2_sampled_full():
    c = WL.config2()
    B = c["logits"].shape[0]
    pol = [J.policy(**c["policy"])] * B
    g, r = both(c["V"], pol, logits=c["logits"], histories=c["histories"],
                generated=c["generated"], uniforms=c["uniforms"], kept_capacity=64)
    assert_same(g, r)
    assert np.all(g["kept_counts"] <= 50) and np.all(g["kept_counts"] >= 1)


@pytest.mark.parametrize("sampled", [False, True])
def test_c3_grammar(sampled):
    c = WL.config3()
    B = c["logits_bf16"].shape[0]
    p = J.policy(temperature=1.0, constrained=True) if sampled else J.policy(constrained=True)
    g, r = both(c["V"], [p] * B, logits_bf16=c["logits_bf16"], masks=c["masks"],
                uniforms=c["uniforms"], kept_capacity=4096 if sampled else 0)
    assert_same(g, r)
    for row in range(B):  # every selected token is admitted by the mask
        assert c["allowed"][row, g["tokens"][row]]


def test_c5_large_full():
    c = WL.config5()
    B = c["logits_bf16"].shape[0]
    pol = [J.policy(**c["policy"])] * B
    g, r = both(c["V"], pol, logits_bf16=c["logits_bf16"], histories=c["histories"],
                generated=c["generated"], mark_prompt=[True] * B,
                uniforms=c["uniforms"], kept_capacity=1024)
    assert_same(g, r)


def rand_logits(rng, rows, V, scale=2.0, decimals=None):
    x = rng.normal(0, scale, (rows, V)).astype(np.float32)
    if decimals is not None:
        x = np.round(x, decimals).astype(np.float32)
    return x


@pytest.mark.parametrize("V", [100, 4097, 8192, 70001, 151936])
def test_mixed_batch_shapes(V):
    rng = np.random.default_rng(V)
    rows = 12
    x = rand_logits(rng, rows, V, decimals=1)
    pols = [J.policy(), J.policy(temperature=0.7, top_k=50, top_p=0.9),
            J.policy(temperature=1.3, top_k=5), J.policy(temperature=0.5, min_p=0.1),
            J.policy(temperature=1.0, top_k=20, min_p=0.2, top_p=0.5),
            J.policy(repetition=1.3), J.policy(temperature=0.9, top_k=1),
            J.policy(temperature=2.0, top_k=300, top_p=0.99),
            J.policy(temperature=0.7, top_k=V + 5, min_p=0.5),
            J.policy(temperature=1.0, top_k=1000), J.policy(temperature=0.3, top_k=64, min_p=1.0),
            J.policy(temperature=0.7, top_k=50, presence=1.5, frequency=-0.5, repetition=0.8)]
    hist = [rng.integers(0, V, 300).astype(np.uint32) for _ in range(rows)]
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, pols, logits=x, histories=hist, generated=[150] * rows,
                mark_prompt=[True] * rows, uniforms=u, kept_capacity=1100)
    assert_same(g, r)


def test_ties_and_constant_rows():
    rng = np.random.default_rng(11)
    V = 20000
    x = np.zeros((6, V), np.float32)
    x[1] = 1.0
    x[2, ::7] = 3.0
    x[3] = np.round(rng.normal(0, 0.5, V), 0)
    x[4] = -0.0
    x[4, ::2] = 0.0
    x[5] = rand_logits(rng, 1, V, decimals=0)[0]
    pols = [J.policy(temperature=1.0, top_k=50), J.policy(temperature=0.5, top_k=300, top_p=0.3),
            J.policy(temperature=1.0, top_k=1000), J.policy(temperature=0.8, top_k=7, top_p=0.9),
            J.policy(temperature=1.0, top_k=33), J.policy()]
    u = np.array([0.1, 0.5, 0.99, 0.0, 0.7, 0.3], np.float32)
    g, r = both(V, pols, logits=x, uniforms=u, kept_capacity=1024)
    assert_same(g, r)


def test_masks_stops_and_sentinels():
    rng = np.random.default_rng(12)
    V = 50000
    rows = 8
    x = rand_logits(rng, rows, V)
    allowed = rng.random((rows, V)) < 0.05
    allowed[0] = False                       # nothing admitted
    x[1] = np.nan                            # NaN row
    x[2] = -np.inf                           # -inf row
    x[3, 123] = np.inf                       # +inf in a sampled row
    x[4, ::3] = np.nan                       # partial NaN
    allowed[5] = False
    allowed[5, [7, 8]] = True                # only the stop tokens
    masks = WL.mask_words(allowed)
    stop = (7, 8)
    pols = [J.policy(constrained=True), J.policy(temperature=1.0), J.policy(temperature=1.0),
            J.policy(temperature=1.0), J.policy(temperature=0.9, top_k=40, constrained=True),
            J.policy(temperature=1.0, constrained=True, exclude_stop=True),
            J.policy(constrained=True, exclude_stop=True), J.policy()]
    x[7] = -np.inf
    x[7, 999] = 5.0
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, pols, logits=x, masks=masks, uniforms=u, stop=stop, kept_capacity=2500)
    assert_same(g, r)
    assert g["tokens"][0] == NO and g["tokens"][1] == NO and g["tokens"][2] == NO
    assert g["tokens"][3] == NO and g["tokens"][5] == NO
    assert g["tokens"][7] == 999


def test_extra_verify_tokens_and_sparse_draft():
    """Verify rows: each row r counts the draft tokens 1..r (penalize_verify)
    and drafted rows draw the residual against 16 sparse candidates."""
    rng = np.random.default_rng(13)
    V = 30000
    rows = 8
    x = rand_logits(rng, rows, V)
    inputs = rng.integers(0, V, rows + 1).astype(np.uint32)
    inputs[3] = inputs[5]  # a repeated draft token
    hist = [rng.integers(0, V, 200).astype(np.uint32)] * rows
    extra = [inputs[1:r + 1] for r in range(rows)]
    cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
    cand[:, 0] = inputs[1:rows + 1]
    cand[2, 5] = cand[2, 0]  # duplicate candidate: first entry counts
    cp = rng.dirichlet(np.ones(16), rows).astype(np.float32)
    p = J.policy(temperature=0.9, top_k=40, top_p=0.95, repetition=1.2, presence=0.4, frequency=0.2)
    u = rng.random(rows).astype(np.float32)
    # make drafts likely kept: boost them
    for r in range(rows):
        x[r, inputs[r + 1]] += 6.0
    g, r = both(V, [p] * rows, logits=x, histories=hist, generated=[100] * rows,
                mark_prompt=[True] * rows, extra=extra, uniforms=u,
                draft_tokens=inputs[1:], drafted_rows=rows - 1,
                cand_ids=cand, cand_probs=cp, kept_capacity=64)
    assert_same(g, r)
    assert np.any(g["draft_probs"][:rows - 1] > 0)


@pytest.mark.parametrize("bf16", [False, True])
def test_extra_tokens_on_the_fast_path(bf16):
    """Verify rows' extra penalty tokens (penalize_verify, sampling.metal:
    978-993) taken by the single fast pass: extras equal to history tokens
    (their fixed slot's count grows), extras with no table entry (penalized
    in place with their own count), repeated extras, extras in the partial
    last chunk, refused by the mask, equal to the stop tokens, and 16 extras
    in one row; greedy, cut and uncut sampled rows, drafted and not. Tokens,
    kept sets and probabilities bit-exact."""
    rng = np.random.default_rng(81 + bf16)
    V = 5 * 8192 + 1234
    rows = 12
    x = rand_logits(rng, rows, V, scale=2.0)
    hist = [rng.integers(0, V, 300).astype(np.uint32) for _ in range(rows)]
    extra = []
    for r in range(rows):
        n = [0, 1, 3, 16, 5, 8, 2, 16, 4, 7, 9, 11][r]
        e = rng.integers(0, V, n).astype(np.uint32)
        if n >= 3:
            e[0] = hist[r][5]                 # a history token: its slot counts it
            e[1] = e[2] = np.argmax(x[r])     # repeated, at the row's best token
        if n >= 5:
            e[3] = V - 3                      # the partial last chunk
            e[4] = 7                          # a stop token
        extra.append(e)
        for t in e:                            # make extras matter: near the top
            x[r, t] = max(x[r, t], np.float32(5.0) + np.float32(rng.random()))
    allowed = rng.random((rows, V)) < 0.6
    allowed[:, 7] = True
    allowed[5, extra[5][5]] = False            # an extra the mask refuses
    pols = [J.policy(repetition=1.3, presence=0.5, frequency=0.4),
            J.policy(temperature=0.8, top_k=40, top_p=0.9, repetition=1.2, presence=0.3),
            J.policy(temperature=1.0, presence=0.8, frequency=0.5),          # uncut
            J.policy(temperature=0.7, top_k=20, repetition=1.1, frequency=1.5),
            J.policy(temperature=0.9, top_k=60, top_p=0.95, presence=2.0, exclude_stop=True),
            J.policy(temperature=0.8, top_k=30, repetition=1.4, constrained=True),
            J.policy(repetition=1.5, presence=1.0, constrained=True),
            J.policy(temperature=1.2, min_p=0.02, top_k=200, presence=0.5, frequency=0.5),
            J.policy(temperature=0.6, top_k=50, top_p=0.8, repetition=0.9, presence=-0.5),
            J.policy(temperature=1.0, repetition=1.2, exclude_stop=True),        # uncut
            J.policy(frequency=2.0, presence=2.0, exclude_stop=True),
            J.policy(temperature=0.75, top_k=10, repetition=1.25, presence=0.2, frequency=0.1)]
    u = rng.random(rows).astype(np.float32)
    d = np.array([int(e[-1]) if len(e) else NO for e in extra], np.uint32)
    cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
    cand[:, 0] = d
    kw = dict(masks=WL.mask_words(allowed), histories=hist, generated=[150] * rows,
              mark_prompt=[True] * rows, extra=extra, uniforms=u, stop=(7, 9),
              draft_tokens=d, drafted_rows=rows, cand_ids=cand,
              cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32),
              kept_capacity=256)
    if bf16:
        kw["logits_bf16"] = WL.to_bf16_bits(x)
    else:
        kw["logits"] = x
    g, r = both(V, pols, **kw)
    assert_same(g, r)


@pytest.mark.parametrize("V", [24 * 8192, 32 * 8192, 248320])
def test_small_merge_refetches_long_lists(V):
    """Rows with top-k 50 and no min-p over 24, 32 and 30.3 chunks (a partial
    last chunk of 2,560 tokens): the small merge's wide fetch (floor(5120 /
    S) slots a chunk, the rest to the last chunk), and where a list passes
    its slots, the compact refetch of the candidates of the chunks that
    reach the row's threshold. Drafted rows with sparse candidates and
    penalized rows among them; bit-exact with the oracle."""
    rng = np.random.default_rng(V % 1000)
    rows = 16
    x = rand_logits(rng, rows, V, scale=2.5)
    pols = [J.policy(temperature=0.7, top_k=50, top_p=0.9, presence=0.5, frequency=0.3)
            if r % 2 else J.policy(temperature=0.9, top_k=40) for r in range(rows)]
    hist = [rng.integers(0, V, 600).astype(np.uint32) for _ in range(rows)]
    d = rng.integers(0, V, rows).astype(np.uint32)
    d[::3] = NO
    cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
    cand[:, 0] = d
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, pols, logits=x, histories=hist, generated=[300] * rows,
                mark_prompt=[False] * rows, uniforms=u, draft_tokens=d, drafted_rows=rows,
                cand_ids=cand, cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32),
                kept_capacity=64)
    assert_same(g, r)


def test_small_merge_refetches_a_long_inner_list():
    """A long list in a chunk other than the last (the last chunk's list also
    gets the fetch's spare slots): chunk 3 of each row holds 320 high,
    distinct values in the registers of its first 10 threads, so few lane
    maxima reach them and the chunk's bound admits all 320. The merge then
    refetches compactly; the rank selection still succeeds (no ties)."""
    rng = np.random.default_rng(77)
    V, rows = 248320, 8
    x = rand_logits(rng, rows, V, scale=1.0)
    # fp32 token c * 8192 + j * 1024 + t * 4 + e sits in thread t's register
    # j * 4 + e.
    toks = np.array([3 * 8192 + j * 1024 + t * 4 + e
                     for j in range(8) for t in range(10) for e in range(4)])
    for r in range(rows):
        x[r, toks] = rng.permutation(np.linspace(3.5, 6.0, toks.size)).astype(np.float32)
    pols = [J.policy(temperature=0.7, top_k=50, top_p=0.9, presence=0.5, frequency=0.3)
            if r % 2 else J.policy(temperature=0.9, top_k=40) for r in range(rows)]
    hist = [rng.integers(0, V, 600).astype(np.uint32) for _ in range(rows)]
    d = rng.integers(0, V, rows).astype(np.uint32)
    d[::3] = NO
    cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
    cand[:, 0] = d
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, pols, logits=x, histories=hist, generated=[300] * rows,
                mark_prompt=[False] * rows, uniforms=u, draft_tokens=d, drafted_rows=rows,
                cand_ids=cand, cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32),
                kept_capacity=64)
    assert_same(g, r)


def test_small_topk_with_many_ties_at_the_kth_key():
    """Rows with top-k <= 64 whose boundary holds hundreds of tied tokens
    spread over the chunks (the one-wave merge's exact top-k by radix and id
    descent), plus rows that just fit and just miss its slot budget."""
    rng = np.random.default_rng(31)
    V = 70000
    rows = 6
    x = rng.normal(0, 1.0, (rows, V)).astype(np.float32)
    tied = rng.choice(V, 500, replace=False)
    top = rng.choice(V, 10, replace=False)
    x[:, tied] = 3.0
    x[:, top] = 5.0
    x[3] = np.round(x[3], 1)
    x[4, :] = np.where(np.arange(V) % 3 == 0, 2.0, -1.0).astype(np.float32)
    x[5, top] = 7.0
    pols = [J.policy(temperature=1.0, top_k=20), J.policy(temperature=0.8, top_k=64, top_p=0.7),
            J.policy(temperature=1.2, top_k=11, min_p=0.01), J.policy(temperature=1.0, top_k=33),
            J.policy(temperature=1.0, top_k=50), J.policy(temperature=0.5, top_k=12)]
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, pols, logits=x, uniforms=u, kept_capacity=64)
    assert_same(g, r)


@pytest.mark.parametrize("bf16,drafted", [(False, False), (True, False), (False, True)])
def test_small_topk_edge_rows(bf16, drafted):
    """Launches whose sampled rows all keep at most 64 tokens (the small-K
    merge): constant rows and rows tied everywhere (overflowing chunks, the
    general path), -inf and NaN rows, penalties, a greedy row, sparse drafts,
    and a partial last chunk, in fp32 and bf16."""
    rng = np.random.default_rng(41 + bf16 + 2 * drafted)
    V = 3 * 8192 + 100
    rows = 10
    x = rand_logits(rng, rows, V)
    x[0] = 1.0
    x[1] = -np.inf
    x[1, [5, 9000, V - 1]] = [0.5, 1.5, -2.0]
    x[4] = np.round(x[4], 1)
    x[5, ::2] = np.nan
    x[6] = np.where(np.arange(V) % 3 == 0, 2.0, -1.0)
    x[9] = np.nan
    hist = [rng.integers(0, V, 300).astype(np.uint32) for _ in range(rows)]
    pols = [J.policy(temperature=1.0, top_k=64), J.policy(temperature=0.9, top_k=50),
            J.policy(temperature=0.8, top_k=40, top_p=0.9, presence=0.3, frequency=0.2),
            J.policy(repetition=1.4), J.policy(temperature=1.1, top_k=64, min_p=0.05),
            J.policy(temperature=1.0, top_k=16), J.policy(temperature=1.0, top_k=33, presence=0.5),
            J.policy(temperature=0.7, top_k=1), J.policy(temperature=1.0, top_k=20, top_p=0.6),
            J.policy(temperature=1.0, top_k=8)]
    u = rng.random(rows).astype(np.float32)
    kw = dict(histories=hist, generated=[200] * rows, mark_prompt=[True] * rows, uniforms=u,
              kept_capacity=64)
    if drafted:
        draft = rng.integers(0, V, rows).astype(np.uint32)
        draft[6] = 3 * 7  # a tied token
        cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
        cand[:, 0] = draft
        kw.update(draft_tokens=draft, drafted_rows=rows - 1, cand_ids=cand,
                  cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32))
    if bf16:
        kw["logits_bf16"] = WL.to_bf16_bits(x)
    else:
        kw["logits"] = x
    g, r = both(V, pols, **kw)
    assert_same(g, r)
    assert g["tokens"][9] == NO


def test_small_topk_over_row_groups():
    """More rows than one selection launch carries (256 rows per launch):
    the row groups' summaries meet in one merge."""
    rng = np.random.default_rng(43)
    V = 9000
    rows = 300
    x = rand_logits(rng, rows, V, decimals=1)
    hist = [rng.integers(0, V, 50).astype(np.uint32) for _ in range(rows)]
    pols = [J.policy(temperature=0.9, top_k=10, top_p=0.8, presence=0.2) if i % 7 else
            J.policy(repetition=1.2) for i in range(rows)]
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, pols, logits=x, histories=hist, generated=[20] * rows,
                mark_prompt=[True] * rows, uniforms=u, kept_capacity=16)
    assert_same(g, r)


@pytest.mark.parametrize("bf16", [False, True])
def test_overflowing_chunks_reselected(bf16):
    """Chunks with more than 1024 candidates (flat or tied values) are
    selected again by the merge with the row's thresholds: penalties,
    verify-row extras and ties at the K-th key all go through that path."""
    rng = np.random.default_rng(21)
    V = 3 * 8192 + 777
    rows = 6
    x = np.round(rng.normal(0, 0.05, (rows, V)), 1).astype(np.float32)
    x[1] = 2.0
    x[2, ::5] = 4.0
    x[3, :9000] = 1.5
    x[4] = np.round(rng.normal(0, 0.02, V), 2)
    hist = [rng.integers(0, V, 3000).astype(np.uint32) for _ in range(rows)]
    extra = [rng.integers(0, V, r).astype(np.uint32) for r in range(rows)]
    pols = [J.policy(temperature=1.0, top_k=64, repetition=1.3, presence=0.2),
            J.policy(temperature=0.7, top_k=500, top_p=0.8, frequency=0.1),
            J.policy(temperature=1.0, top_k=1000, presence=0.5),
            J.policy(temperature=0.9, top_k=200, min_p=0.5, repetition=0.8),
            J.policy(temperature=1.2, top_k=1024, top_p=0.99),
            J.policy(temperature=1.0, top_k=3, presence=-0.4)]
    u = rng.random(rows).astype(np.float32)
    kw = dict(histories=hist, generated=[1500] * rows, mark_prompt=[True] * rows,
              extra=extra, uniforms=u, kept_capacity=1024)
    if bf16:
        kw["logits_bf16"] = WL.to_bf16_bits(x)
    else:
        kw["logits"] = x
    g, r = both(V, pols, **kw)
    assert_same(g, r)


@pytest.mark.parametrize("kind", ["unfiltered", "topp", "minp", "bigk", "all"])
def test_multipass_stages(kind):
    rng = np.random.default_rng(14)
    V = 151936 if kind in ("unfiltered", "topp") else 60000
    rows = 4
    x = rand_logits(rng, rows, V, scale=1.0)
    pol = {"unfiltered": J.policy(temperature=1.0),
           "topp": J.policy(temperature=0.8, top_p=0.9),
           "minp": J.policy(temperature=1.0, min_p=0.02),
           "bigk": J.policy(temperature=1.5, top_k=5000),
           "all": J.policy(temperature=0.9, top_k=3000, top_p=0.7, min_p=0.01)}[kind]
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, [pol] * rows, logits=x, uniforms=u, kept_capacity=V)
    assert_same(g, r)


@pytest.mark.parametrize("bf16,greedy,draft", [(False, True, None), (True, True, None),
                                               (False, False, None), (False, True, "dense"),
                                               (True, False, "dense"), (False, True, "sparse")])
def test_unfiltered_mass_draw(bf16, greedy, draft):
    """Launches whose sampled rows keep every admitted token and carry no
    draft, without kept outputs: chunk maxima, then the mass-and-draw launch
    (greedy rows ride along). Penalties, masks, stop exclusion, a partial
    last chunk, the sentinel rows and uniforms at both ends."""
    rng = np.random.default_rng(61 + bf16)
    V = 8 * 8192 + 4465
    rows = 12
    x = rand_logits(rng, rows, V, scale=1.5)
    allowed = rng.random((rows, V)) < 0.3
    x[1] = np.nan                             # nothing admitted: sentinel
    x[2] = -np.inf                            # no mass: sentinel
    x[3, 123] = np.inf                        # +inf maximum: sentinel
    x[4, ::3] = np.nan                        # NaN tokens are never drawn
    allowed[5] = False
    allowed[5, [7, 8, 40000]] = True          # the stop tokens and one other
    x[6] = -80.0
    x[6, V - 1] = 3.0                         # the partial chunk's last token
    x[6, 5] = 2.9
    x[10] = np.round(x[10], 0)                # ties everywhere
    masks = WL.mask_words(allowed)
    hist = [rng.integers(0, V, 500).astype(np.uint32) for _ in range(rows)]
    hist[11] = np.concatenate([hist[11], np.full(900, 4321, np.uint32)])
    pols = [J.policy(temperature=1.0, constrained=True), J.policy(temperature=1.0),
            J.policy(temperature=0.8), J.policy(temperature=1.0),
            J.policy(temperature=0.7, presence=0.4, frequency=0.2),
            J.policy(temperature=1.0, constrained=True, exclude_stop=True),
            J.policy(temperature=0.25), J.policy(constrained=True, repetition=1.2),
            J.policy(), J.policy(temperature=2.0, repetition=1.3),
            J.policy(temperature=1.0), J.policy(temperature=1.5, presence=1.0, frequency=0.5)]
    if not greedy:  # every row sampled: the chunk loads go out first
        pols[7] = J.policy(temperature=1.0, constrained=True, repetition=1.2)
        pols[8] = J.policy(temperature=3.0)
    u = rng.random(rows).astype(np.float32)
    u[0] = 0.0
    u[9] = np.float32(1.0) - np.float32(2.0 ** -24)
    kw = dict(masks=masks, histories=hist, generated=[300] * rows,
              mark_prompt=[True] * rows, uniforms=u, stop=(7, 8))
    if draft is not None:
        # Drafted rows draw the residual max(p - q, 0): drafts at the row's
        # best token (mass left only if q is small there), at a token the
        # mask refuses, and at random tokens; two rows carry no draft.
        d = rng.integers(0, V, rows).astype(np.uint32)
        d[0] = int(np.nanargmax(np.where(allowed[0], x[0], -np.inf)))
        d[5] = 9                              # refused by row 5's mask
        d[[4, 9]] = NO
        kw.update(draft_tokens=d, drafted_rows=rows)
        if draft == "dense":
            q = rng.dirichlet(np.ones(V) * 0.2, rows).astype(np.float32)
            q[2] = 0.0
            q[10, d[10]] = 1.0                # residual without mass at its draft
            kw["dense_q"] = q
        else:
            cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
            cand[:, 0] = d
            kw.update(cand_ids=cand, cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32))
    if bf16:
        kw["logits_bf16"] = WL.to_bf16_bits(x)
    else:
        kw["logits"] = x
    g, r = both(V, pols, **kw)
    assert_same(g, r)
    assert all(g["tokens"][k] == NO for k in (1, 2, 3))
    assert g["tokens"][5] == 40000            # the one token row 5 admits
    assert g["tokens"][8] != NO and g["tokens"][0] != NO


@pytest.mark.parametrize("kind", ["small", "general", "staged", "drafted"])
def test_mixed_cut_and_uncut_rows(kind):
    """Launches mixing rows with a cut and rows that keep every admitted
    token: the merge (small, general, or with stages for a large k) finishes
    the cut rows and greedy rows, the mass-and-draw launch the uncut ones."""
    rng = np.random.default_rng(71 + len(kind))
    V = 5 * 8192 + 1234
    rows = 10
    x = rand_logits(rng, rows, V, scale=2.0)
    x[3, ::5] = np.nan
    allowed = rng.random((rows, V)) < 0.4
    masks = WL.mask_words(allowed)
    cut = {"small": J.policy(temperature=0.8, top_k=50, top_p=0.9),
           "general": J.policy(temperature=0.8, top_k=300, top_p=0.9),
           "staged": J.policy(temperature=1.1, top_k=3000, min_p=0.01),
           "drafted": J.policy(temperature=0.9, top_k=40)}[kind]
    pols = [cut, J.policy(temperature=1.0), J.policy(), J.policy(temperature=0.6, presence=0.3),
            cut, J.policy(temperature=1.0, constrained=True), J.policy(temperature=0.7, top_k=20),
            J.policy(temperature=1.3, repetition=1.2), J.policy(constrained=True),
            J.policy(temperature=1.0)]
    hist = [rng.integers(0, V, 400).astype(np.uint32) for _ in range(rows)]
    u = rng.random(rows).astype(np.float32)
    kw = dict(masks=masks, histories=hist, generated=[200] * rows,
              mark_prompt=[True] * rows, uniforms=u, logits=x)
    if kind == "drafted":
        d = rng.integers(0, V, rows).astype(np.uint32)
        d[[2, 8]] = NO
        cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
        cand[:, 0] = d
        kw.update(draft_tokens=d, drafted_rows=rows, cand_ids=cand,
                  cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32))
    g, r = both(V, pols, **kw)
    assert_same(g, r)
    assert np.all(g["tokens"] != NO)


def _uncut_rows(rng, rows, V, uniform):
    """Rows that keep every admitted token, with masks, stop exclusion and
    the sentinel cases, for the draw finished in the select launch."""
    x = rand_logits(rng, rows, V, scale=1.5)
    allowed = rng.random((rows, V)) < 0.3
    allowed[:, :40] = True
    if rows >= 8:
        allowed[3, 123] = True
        x[1] = np.nan                         # nothing admitted: sentinel
        x[2] = -np.inf                        # no mass: sentinel
        x[3, 123] = np.inf                    # +inf maximum: sentinel
        x[4, ::3] = np.nan                    # NaN tokens are never drawn
        allowed[5] = False
        allowed[5, [7, 8, V - 2]] = True      # the stop tokens and one other
        x[6] = -60.0
        x[6, V - 1] = 3.0                     # the last chunk's last token
        x[6, 5] = 2.5
        x[7] = np.round(x[7], 0)              # ties everywhere
    masks = WL.mask_words(allowed)
    if uniform:
        pols = [J.policy(temperature=1.0, constrained=True, exclude_stop=True)] * rows
    else:
        temps = [1.0, 1.0, 0.8, 1.0, 0.7, 1.0, 0.25, 1.3, 3.0, 0.5]
        pols = [J.policy(temperature=temps[r % 10], constrained=r % 3 != 1,
                         exclude_stop=r % 2 == 1) for r in range(rows)]
    u = rng.random(rows).astype(np.float32)
    u[0] = 0.0
    u[rows - 1] = np.float32(1.0) - np.float32(2.0 ** -24)
    return x, masks, pols, u


# Vocabularies whose rows stay 16-byte aligned (the fast kernel's launches).
@pytest.mark.parametrize("bf16,uniform,V", [(False, True, 5 * 8192 + 1240),
                                            (True, True, 5 * 8192 + 1240),
                                            (False, False, 19 * 8192 - 4),
                                            (True, False, 3000)])
def test_rows_with_no_cut_drawn_in_the_select_launch(bf16, uniform, V):
    """Launches whose rows all keep every admitted token, with no draft,
    penalty or kept output: each row's last chunk block gathers the other
    chunks' self-validating summaries and draws (no uncut_kernel launch).
    Uniform and per-row policies, fp32 and bf16, a partial last chunk, one
    chunk only; bit-exact with the oracle."""
    rng = np.random.default_rng(V + 2 * bf16 + uniform)
    rows = 10
    x, masks, pols, u = _uncut_rows(rng, rows, V, uniform)
    kw = dict(masks=masks, uniforms=u, stop=(7, 8))
    kw["logits_bf16" if bf16 else "logits"] = WL.to_bf16_bits(x) if bf16 else x
    g, r = both(V, pols, **kw)
    assert_same(g, r)
    assert all(g["tokens"][k] == NO for k in (1, 2, 3))
    assert g["tokens"][0] != NO


def test_rows_with_no_cut_across_calls_on_one_sampler():
    """The in-launch draw's summary words are returned to zero by each call's
    finisher: calls of 10, 3 and 10 rows with new inputs on one sampler,
    each bit-exact with the oracle."""
    rng = np.random.default_rng(91)
    V = 7 * 8192 + 100
    s = J.Sampler(V, 10)
    for rows in (10, 3, 10, 10):
        x, masks, pols, u = _uncut_rows(rng, rows, V, uniform=rows == 3)
        kw = dict(masks=masks, uniforms=u, stop=(7, 8), logits=x)
        print(f"call rows={rows}", flush=True)
        g = run_gpu(V, pols, sampler=s, **kw)
        r = run_oracle(V, pols, **kw)
        assert_same(g, r)


def test_c3_sampled_without_kept_outputs():
    """C3 sampled as the engine calls it (no kept outputs): the draw finished
    in the select launch, at full size."""
    c = WL.config3()
    B = c["logits_bf16"].shape[0]
    p = J.policy(temperature=1.0, constrained=True)
    g, r = both(c["V"], [p] * B, logits_bf16=c["logits_bf16"], masks=c["masks"],
                uniforms=c["uniforms"])
    assert_same(g, r)
    for row in range(B):
        assert c["allowed"][row, g["tokens"][row]]


def test_dense_residual_multipass():
    rng = np.random.default_rng(15)
    V = 40000
    rows = 4
    x = rand_logits(rng, rows, V)
    q = rng.dirichlet(np.ones(V) * 0.3, rows).astype(np.float32)
    d = np.array([int(np.argmax(x[r])) for r in range(rows)], np.uint32)
    d[3] = 17
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, [J.policy(temperature=1.0)] * rows, logits=x, uniforms=u,
                draft_tokens=d, dense_q=q, kept_capacity=0)
    assert_same(g, r)


@pytest.mark.parametrize("bf16", [False, True])
def test_dense_residual_in_the_partial_last_chunk(bf16):
    """The last row's residual draw lands in the partial last chunk (V is not
    a multiple of 8192): its mass sits at V - 1, where q is small, and the
    dense q buffer is exactly rows x V floats, so a read of q past the
    vocabulary would leave the buffer. Tokens and p(draft) bit-exact."""
    rng = np.random.default_rng(29 + bf16)
    V = 151936
    rows = 3
    x = np.full((rows, V), -12.0, np.float32) + rng.random((rows, V), dtype=np.float32)
    x[:, V - 1] = 9.0
    x[:, V - 40:V - 1] += 4.0
    q = rng.dirichlet(np.ones(V), rows).astype(np.float32)
    q[:, V - 1] = 1e-4
    d = np.array([5, V - 2, 77], np.uint32)
    u = np.array([0.3, 0.999, 0.9999], np.float32)
    kw = dict(uniforms=u, draft_tokens=d, dense_q=np.ascontiguousarray(q))
    if bf16:
        kw["logits_bf16"] = WL.to_bf16_bits(x)
    else:
        kw["logits"] = x
    g, r = both(V, [J.policy(temperature=1.0)] * rows, **kw)
    assert_same(g, r)
    assert g["tokens"][rows - 1] >= V - 4480  # inside the partial last chunk


@pytest.mark.parametrize("bf16,sparse", [(False, False), (True, False), (False, True)])
def test_residual_launch_draws_every_row(bf16, sparse):
    """A launch of drafted rows with no cut, penalty or mask (the residual
    pass) beside greedy rows and undrafted rows with no cut, without kept
    lists: the residual launch draws every row (each drafted row in its last
    chunk block to arrive, the others in blocks of their own), with no
    further launch. Rows 0-7 are drafted: a draft in the partial last chunk,
    a q that leaves no residual mass (the plain draw, with p(draft)), a zero
    q row (the residual is p itself), a row of NaN (the sentinel), a drafted
    row whose draft is JF_NO_TOKEN, a draft that is an excluded stop token;
    their q dense, or 16 sparse candidates. Rows 8-13 are not drafted: a
    penalized and a plain greedy row, a masked row, a row of -inf (the
    sentinel) and uniforms at both ends. Bit-exact with the oracle."""
    rng = np.random.default_rng(131 + bf16 + 2 * sparse)
    V = 6 * 8192 + 777
    rows, drafted = 14, 8
    x = rand_logits(rng, rows, V, scale=2.0)
    x[4] = np.nan                              # nothing admitted
    x[7, ::7] = np.nan
    x[12] = -np.inf                            # no mass
    allowed = rng.random((rows, V)) < 0.3
    q = rng.dirichlet(np.ones(V) * 0.3, rows).astype(np.float32)
    q[2] = 1.0                                 # q covers p everywhere: no residual
    q[3] = 0.0                                 # the residual is p
    d = rng.integers(0, V, rows).astype(np.uint32)
    d[1] = V - 3                               # in the partial last chunk
    d[5] = NO
    pols = [J.policy(temperature=T) for T in (1.0, 0.7, 1.0, 1.5, 1.0, 0.9)]
    pols += [J.policy(temperature=1.0, exclude_stop=True), J.policy(temperature=2.0)]
    pols += [J.policy(repetition=1.3), J.policy(),
             J.policy(temperature=0.8, constrained=True), J.policy(temperature=1.2),
             J.policy(temperature=1.0), J.policy(temperature=0.5)]
    hist = [rng.integers(0, V, 300).astype(np.uint32) for _ in range(rows)]
    u = rng.random(rows).astype(np.float32)
    u[0] = 0.0
    u[13] = np.float32(1.0) - np.float32(2.0 ** -24)
    kw = dict(masks=WL.mask_words(allowed), histories=hist, generated=[100] * rows,
              mark_prompt=[True] * rows, uniforms=u, stop=(int(d[6]), 17),
              draft_tokens=d, drafted_rows=drafted)
    if sparse:
        cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
        cand[:, 0] = d
        cand[1, 3] = V - 1
        kw.update(cand_ids=cand, cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32))
    else:
        kw["dense_q"] = q
    kw["logits_bf16" if bf16 else "logits"] = WL.to_bf16_bits(x) if bf16 else x
    g, r = both(V, pols, **kw)
    assert_same(g, r)
    assert g["tokens"][4] == NO and g["tokens"][12] == NO
    assert g["tokens"][6] != d[6]              # the stop token is excluded
    assert g["draft_probs"][2] > 0.0


def test_residual_launches_over_many_rows():
    """More rows than one residual launch holds (256): drafted rows with no
    cut (some with JF_NO_TOKEN drafts) interleaved with greedy rows, then
    undrafted rows, two vocabulary chunks a row; every launch draws its own
    rows."""
    rng = np.random.default_rng(137)
    V = 2 * 8192 + 100
    rows = 300
    x = rand_logits(rng, rows, V, scale=1.5)
    q = rng.dirichlet(np.ones(V) * 0.5, rows).astype(np.float32)
    d = rng.integers(0, V, rows).astype(np.uint32)
    d[::11] = NO
    pols = [J.policy() if k % 5 == 4 else J.policy(temperature=0.6 + 0.1 * (k % 7))
            for k in range(rows)]
    u = rng.random(rows).astype(np.float32)
    g, r = both(V, pols, logits=x, uniforms=u, draft_tokens=d, drafted_rows=200, dense_q=q)
    assert_same(g, r)


FAR_OFFSETS = [0, 5, 10, 15, 20, 22, 30, 45, 60, 80]


def far_row(rng, T, shift):
    """One row whose chunk c holds values up to 4 T below
    3 - FAR_OFFSETS[(c + shift) % 10] T (the row maximum 3 in one chunk), a
    partial last chunk, and four tokens at 3 - 82 T."""
    C = len(FAR_OFFSETS)
    V = C * 8192 + 333
    x = np.empty(V, np.float32)
    offs = np.roll(FAR_OFFSETS, shift)
    for c in range(C + 1):
        lo, hi = c * 8192, min((c + 1) * 8192, V)
        d = offs[c] if c < C else 3
        x[lo:hi] = 3.0 - d * T - 4.0 * T * rng.random(hi - lo)
        x[lo + int(rng.integers(0, hi - lo))] = 3.0 - d * T
    x[rng.integers(0, V, 4)] = 3.0 - 82.0 * T
    return V, x


def assert_softmax_close(got, want):
    """1e-5 relative where the probability is a normal float with margin;
    below that the reported value is either 0 (flushed under FLT_MIN) or
    within the same bound."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    ok = (np.abs(got - want) <= 1e-5 * want) | ((want < 1e-36) & (got == 0))
    assert ok.all(), (got[~ok][:5], want[~ok][:5])


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("draft", [None, "sparse", "dense"])
def test_far_chunk_offsets_report_softmax_probabilities(bf16, draft):
    """Rows with no cut whose chunk maxima sit 0 to 80 T below the row maximum
    (tokens to 84 T): tokens, kept probabilities and p(draft) bit-exact with
    the oracle, and every reported probability within 1e-5 relative of
    float64 softmax (sampling.metal:38-40, 647-652, 828-829). Masked rows take
    the general uncut pass (kept outputs, sparse drafts); unmasked rows with a
    dense q take the lean residual pass. Drafts sit in chunks whose offsets
    differ by row."""
    rng = np.random.default_rng(91 + 2 * bf16 + (draft == "dense"))
    rows = 6
    T = [0.7, 1.0, 2.0] * 2
    xs = []
    for r in range(rows):
        V, x = far_row(rng, T[r], r)
        xs.append(x)
    x = np.stack(xs)
    if bf16:
        lg = WL.to_bf16_bits(x)
        x = (lg.astype(np.uint32) << 16).view(np.float32)
    else:
        lg = x
    masked = draft != "dense"
    allowed = np.ones((rows, V), bool)
    if masked:
        allowed = rng.random((rows, V)) < 0.002
        allowed[:, ::4096] = True
    pols = [J.policy(temperature=T[r], constrained=masked) for r in range(rows)]
    u = rng.random(rows).astype(np.float32)
    kw = dict(uniforms=u, kept_capacity=512 if masked else 0)
    kw["logits_bf16" if bf16 else "logits"] = lg
    if masked:
        kw["masks"] = WL.mask_words(allowed)
    if draft is not None:
        d = np.empty(rows, np.uint32)
        for r in range(rows):
            c = (3 * r + 1) % 10
            d[r] = c * 8192 + int(rng.choice(np.flatnonzero(allowed[r, c * 8192:(c + 1) * 8192])))
        kw.update(draft_tokens=d, drafted_rows=rows)
        if draft == "dense":
            kw["dense_q"] = rng.dirichlet(np.ones(V) * 0.5, rows).astype(np.float32)
        else:
            cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
            cand[:, 0] = d
            kw.update(cand_ids=cand,
                      cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32))
    g, r = both(V, pols, **kw)
    assert_same(g, r)
    for k in range(rows):
        ref = softmax_rows(x[k:k + 1], allowed[k:k + 1], T[k])[0]
        if masked:
            n = int(r["kept_counts"][k])
            assert n == int(allowed[k].sum()) and n <= 512
            assert_softmax_close(g["kept_probs"][k, :n], ref[r["kept_ids"][k, :n]])
        if draft is not None:
            assert_softmax_close([g["draft_probs"][k]], [ref[int(kw["draft_tokens"][k])]])


def softmax_rows(x, allowed, T):
    out = np.zeros(x.shape)
    for r in range(x.shape[0]):
        v = np.where(allowed[r], x[r].astype(np.float64), -np.inf)
        e = np.exp((v - v.max()) / float(np.float32(T)))
        out[r] = e / e.sum()
    return out


def test_greedy_rows_across_two_launches():
    """300 greedy rows: two launches of the fast kernel (256 rows, then 44),
    each row finished by its last chunk block waiting for the row's other
    blocks; maxima tied across chunks in some rows (lowest id wins). Three
    calls on one sampler (the words return to zero between them); tokens
    equal the oracle's."""
    from harness import run_gpu, run_oracle
    V = 151936
    rows = 300
    rng = np.random.default_rng(77)
    x = rng.normal(0, 2.0, (rows, V)).astype(np.float32)
    for r in range(0, rows, 7):
        x[r, [r % 8192, V // 2 + r, V - 1 - r]] = 40.0
    pols = [J.policy(repetition=1.0)] * rows
    s = J.Sampler(V, rows)
    g = run_gpu(V, pols, sampler=s, repeat=3, logits=x)
    o = run_oracle(V, pols, logits=x)
    np.testing.assert_array_equal(g["tokens"], o["tokens"])
    assert np.all(g["tokens"][::7] == np.array([r % 8192 for r in range(0, rows, 7)], np.uint32))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("V", [5000, 3 * 8192 + 17, 151936])
def test_all_greedy_launch_edges(bf16, V):
    """Launches whose rows are all greedy finish inside the selection: each
    chunk's best is packed into one word and the row's finishing block (its
    last chunk's) takes the largest (sampling.metal:1427-1512). Ties of the maximum across chunks
    (lowest id), -0 against +0, +inf, all-NaN, all -inf (admitted: it wins
    over nothing), a mask that admits nothing and one that admits only the
    partial last chunk; then calls on the same sampler with fewer rows,
    which find the packed words and counters returned to zero."""
    rng = np.random.default_rng(41 + V)
    rows = 8
    x = rng.normal(0, 2.0, (rows, V)).astype(np.float32)
    x[1, [10, V // 2, V - 1]] = 50.0            # the maximum in three chunks
    x[2] = np.nan
    x[3] = -np.inf
    x[4] = -1.0
    x[4, [V - 2, 3]] = -0.0
    x[4, 7] = 0.0
    x[5, V // 3] = np.inf
    allowed = np.ones((rows, V), bool)
    allowed[6] = False                           # nothing admitted
    allowed[7] = False
    allowed[7, V - 5:] = True                    # only the last few tokens
    masks = WL.mask_words(allowed)
    pols = [J.policy()] * 6 + [J.policy(constrained=True)] * 2
    kw = dict(masks=masks)
    if bf16:
        kw["logits_bf16"] = (x.view(np.uint32) >> 16).astype(np.uint16)
    else:
        kw["logits"] = x
    s = J.Sampler(V, rows)
    g = run_gpu(V, pols, sampler=s, repeat=3, **kw)
    r = run_oracle(V, pols, **kw)
    assert_same(g, r)
    assert g["tokens"][1] == 10 and g["tokens"][2] == NO and g["tokens"][3] == 0
    assert g["tokens"][4] == 3 and g["tokens"][5] == V // 3 and g["tokens"][6] == NO
    assert g["tokens"][7] >= V - 5
    for n in (3, 1):
        sub = {k: v[rows - n:] for k, v in kw.items()}
        g = run_gpu(V, pols[rows - n:], sampler=s, **sub)
        r = run_oracle(V, pols[rows - n:], **sub)
        assert_same(g, r)
    s.close()


def test_determinism_repeat():
    c = WL.config2(B=16)
    pol = [J.policy(**c["policy"])] * 16
    kw = dict(logits=c["logits"], histories=c["histories"], generated=c["generated"],
              uniforms=c["uniforms"][:16], kept_capacity=64)
    a = run_gpu(c["V"], pol, **kw)
    b = run_gpu(c["V"], pol, repeat=3, **kw)
    for k in a:
        np.testing.assert_array_equal(a[k], b[k])


def test_chi_square_of_one_million_draws():
    """1e6 draws of one row (rows share the logits, uniforms differ) against
    the kept distribution."""
    import torch
    from scipy import stats
    V = 256
    rows = 1 << 17
    calls = 8
    rng = np.random.default_rng(16)
    base = rng.normal(0, 1.5, V).astype(np.float32)
    pol = J.policy(temperature=0.8, top_k=40, top_p=0.9)
    dev = torch.device("cuda", 0)
    lg = torch.from_numpy(np.tile(base, (rows, 1))).to(dev)
    out = torch.zeros(rows, dtype=torch.int32, device=dev)
    s = J.Sampler(V, rows)
    gen = torch.Generator(device=dev)
    gen.manual_seed(16)
    toks = []
    for _ in range(calls):
        u = torch.rand(rows, device=dev, generator=gen)
        s.sample(lg, [pol] * rows, out, uniforms=u)
        toks.append(out.cpu().numpy().copy())
    toks = np.concatenate(toks)
    rows = rows * calls
    ref = run_oracle(V, [pol], logits=base[None], uniforms=np.zeros(1, np.float32),
                     kept_capacity=V)
    ids = ref["kept_ids"][0, :ref["kept_counts"][0]]
    probs = ref["kept_probs"][0, :ref["kept_counts"][0]].astype(np.float64)
    assert set(np.unique(toks)) <= set(ids.tolist())
    counts = np.array([(toks == t).sum() for t in ids])
    expected = probs / probs.sum() * rows
    keep = expected >= 5
    chi2 = ((counts[keep] - expected[keep]) ** 2 / expected[keep]).sum()
    pval = stats.chi2.sf(chi2, keep.sum() - 1)
    assert pval > 1e-4, (chi2, pval)


def test_chi_square_two_pass_draw():
    """1e6 draws from rows with no cut (the two-pass draw: chunk masses, then
    slice and token walks) against the float64 softmax of 200 tokens spread
    over two chunks and their wave slices; every other token is -inf."""
    import torch
    from scipy import stats
    V = 2 * 8192
    rows = 4096
    calls = 245
    rng = np.random.default_rng(17)
    ids = np.sort(rng.choice(V, 200, replace=False))
    ids[:3] = [0, 8191, 8192]                # chunk and slice edges
    ids = np.unique(ids)
    base = np.full(V, -np.inf, np.float32)
    base[ids] = rng.uniform(-1.0, 1.0, len(ids)).astype(np.float32)
    pol = J.policy(temperature=1.0)
    dev = torch.device("cuda", 0)
    lg = torch.from_numpy(np.tile(base, (rows, 1))).to(dev)
    out = torch.zeros(rows, dtype=torch.int32, device=dev)
    s = J.Sampler(V, rows)
    gen = torch.Generator(device=dev)
    gen.manual_seed(17)
    counts = torch.zeros(V, dtype=torch.int64, device=dev)
    for _ in range(calls):
        u = torch.rand(rows, device=dev, generator=gen)
        s.sample(lg, [pol] * rows, out, uniforms=u)
        counts += torch.bincount(out.long(), minlength=V)[:V]
    counts = counts.cpu().numpy()
    n = rows * calls
    assert counts.sum() == n
    assert counts[np.setdiff1d(np.arange(V), ids)].sum() == 0   # only weighted tokens
    w = np.exp(base[ids].astype(np.float64))
    expected = w / w.sum() * n
    chi2 = ((counts[ids] - expected) ** 2 / expected).sum()
    pval = stats.chi2.sf(chi2, len(ids) - 1)
    assert pval > 1e-4, (chi2, pval)
