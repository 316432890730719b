"""Seeded random calls of jf_sample against the oracle, bit-exact (tokens,
draft probabilities, kept sets and probabilities). Each call mixes row kinds
the hand-built cases test one at a time: greedy rows, sampled rows with and
without a cut (top-k small and large, top-p, min-p), penalties from uniform
and clustered histories (rows on the fast kernel, rows past its fixed slots,
calls split between the select kernels), masks and stop exclusion, verify
extras, sparse or dense drafts, fp32 and bf16 logits, vocabularies that do
and do not fill a chunk. The seeds are fixed, so a call that passes once
passes again."""
import numpy as np
import pytest

import jf_sampler as J
from jf_sampler import workloads as WL
from harness import NO, assert_same, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def random_call(seed):
    rng = np.random.default_rng(seed)
    V = int(rng.choice([700, 8192, 8193, 20000, 3 * 8192 + 5, 151936]))
    rows = int(rng.integers(1, 25))
    bf16 = bool(rng.random() < 0.4)
    x = (rng.standard_normal((rows, V)) * rng.uniform(0.5, 4.0)).astype(np.float32)
    if rng.random() < 0.3:
        x = np.round(x, 0)  # many ties
    pols, hist, extra = [], [], []
    any_pen = rng.random() < 0.6
    constrained_any = rng.random() < 0.4
    allowed = rng.random((rows, V)) < rng.uniform(0.02, 0.6)
    for r in range(rows):
        kind = rng.integers(0, 5)
        kw = {}
        if kind > 0:
            kw["temperature"] = float(rng.choice([0.3, 0.7, 1.0, 1.6]))
            if kind >= 2:
                kw["top_k"] = int(rng.choice([1, 7, 50, 64, 300, 2000]))
            if kind >= 3 and rng.random() < 0.6:
                kw["top_p"] = float(rng.choice([0.3, 0.9, 0.99]))
            if kind == 4 and rng.random() < 0.6:
                kw["min_p"] = float(rng.choice([0.01, 0.1]))
        h = None
        if any_pen and rng.random() < 0.7:
            kw.update(repetition=float(rng.choice([1.0, 1.2, 0.8])),
                      presence=float(rng.choice([0.0, 0.5, -0.3])),
                      frequency=float(rng.choice([0.0, 0.4])))
            if rng.random() < 0.3:
                h = np.minimum(rng.zipf(1.2, int(rng.integers(200, 3000))) - 1, V - 1)
            else:
                h = rng.integers(0, V, int(rng.integers(1, 1500)))
            h = h.astype(np.uint32)
        if constrained_any and rng.random() < 0.6:
            kw["constrained"] = True
        if rng.random() < 0.2:
            kw["exclude_stop"] = True
        pols.append(J.policy(**kw))
        hist.append(h)
        extra.append(rng.integers(0, V, int(rng.integers(0, 4))).astype(np.uint32)
                     if h is not None and rng.random() < 0.2 else np.zeros(0, np.uint32))
    call = dict(uniforms=rng.random(rows).astype(np.float32),
                stop=(int(rng.integers(0, V)), NO) if rng.random() < 0.5 else (NO, NO))
    if bf16:
        call["logits_bf16"] = WL.to_bf16_bits(x)
    else:
        call["logits"] = x
    if constrained_any:
        call["masks"] = WL.mask_words(allowed)
    if any(h is not None for h in hist):
        call.update(histories=hist,
                    generated=[int(rng.integers(0, len(h))) if h is not None else 0 for h in hist],
                    mark_prompt=[bool(rng.random() < 0.5) for _ in range(rows)])
        if any(len(e) for e in extra):
            call["extra"] = extra
    if rng.random() < 0.4:
        drafted = int(rng.integers(1, rows + 1))
        call.update(draft_tokens=rng.integers(0, V, rows).astype(np.uint32),
                    drafted_rows=drafted)
        if rng.random() < 0.5:
            q = rng.dirichlet(np.ones(V) * 0.05, rows).astype(np.float32)
            call["dense_q"] = q
        else:
            cid = rng.integers(0, V, (rows, 16)).astype(np.uint32)
            cid[:, 0] = call["draft_tokens"]
            call.update(cand_ids=cid,
                        cand_probs=rng.dirichlet(np.ones(16), rows).astype(np.float32))
    if rng.random() < 0.5:
        call["kept_capacity"] = int(rng.choice([16, 64, 256]))
    return V, pols, call


@pytest.mark.parametrize("seed", range(120))
def test_random_mixed_call(seed):
    V, pols, call = random_call(1000 + seed)
    print(f"random call seed={1000 + seed} V={V} rows={len(pols)} keys={sorted(call)}",
          flush=True)
    g = run_gpu(V, pols, **call)
    r = run_oracle(V, pols, **call)
    assert_same(g, r)
