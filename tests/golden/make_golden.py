"""Writes tests/golden/select_cases.{json,npz}: seeded small selection cases
and the outputs the CPU oracle (oracle/jf_oracle.c) gives for them.

The reference ships no golden vectors for this path (its sampler numerics
are pinned by no test), so these fixtures are the oracle's own outputs. They
pin the oracle against regressions (tests/test_golden.py, CPU) and give the
GPU a check that does not depend on building the oracle on the box
(tests/test_golden.py, gpu). Regenerate with

    python tests/golden/make_golden.py

after a deliberate change of the oracle's semantics, and say why in the
commit."""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "justfit-llm_amd"))
sys.path.insert(0, os.path.join(REPO, "oracle"))
sys.path.insert(0, os.path.join(REPO, "tests"))

from jf_sampler import workloads as WL  # noqa: E402

NO = 0xFFFFFFFF


def cases():
    out = []
    # A: fp32, penalties (prompt-marked history on two rows), every filter.
    rng = np.random.default_rng(901)
    V = 3001
    x = rng.normal(0, 2.0, (6, V)).astype(np.float32)
    x[:, rng.choice(V, 5, replace=False)] += 6.0
    hist = [None, rng.integers(0, V, 300).astype(np.uint32), None,
            rng.integers(0, V, 40).astype(np.uint32), None, None]
    pols = [dict(),
            dict(temperature=0.7, top_k=50, top_p=0.9, presence=0.5, frequency=0.3),
            dict(temperature=1.0, min_p=0.1, top_k=200),
            dict(temperature=0.8, top_k=20, repetition=1.2, presence=0.5),
            dict(temperature=1.3, top_p=0.5),
            dict(temperature=0.5, top_k=1)]
    u = rng.random(6).astype(np.float32)
    out.append(dict(name="fp32_filters_penalties", V=V, policies=pols,
                    arrays=dict(logits=x, uniforms=u),
                    histories=hist, generated=[0, 200, 0, 0, 0, 0],
                    mark_prompt=[False, True, False, True, False, False],
                    kept_capacity=256))
    # B: bf16, constraint mask and stop exclusion, sampled and greedy.
    rng = np.random.default_rng(902)
    V = 5000
    x = rng.normal(0, 2.0, (4, V)).astype(np.float32)
    allowed = rng.random((4, V)) < 0.1
    allowed[:, [7, 8]] = True
    pols = [dict(constrained=True), dict(temperature=1.0, constrained=True),
            dict(temperature=0.9, top_k=40, constrained=True, exclude_stop=True),
            dict(exclude_stop=True)]
    x[3, 7] = 50.0
    u = rng.random(4).astype(np.float32)
    out.append(dict(name="bf16_mask_stop", V=V, policies=pols,
                    arrays=dict(logits_bf16=WL.to_bf16_bits(x), masks=WL.mask_words(allowed),
                                uniforms=u),
                    stop=[7, 8], kept_capacity=600))
    # C: drafted rows with 16 sparse candidates (residual draw, p(draft)).
    rng = np.random.default_rng(903)
    V = 2048
    rows = 5
    x = rng.normal(0, 1.5, (rows, V)).astype(np.float32)
    draft = rng.integers(0, V, rows).astype(np.uint32)
    for r in range(rows):
        x[r, draft[r]] += 3.0
    cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
    cand[:, 0] = draft
    cp = rng.dirichlet(np.ones(16), rows).astype(np.float32)
    pols = [dict(temperature=0.9, top_k=40, top_p=0.95)] * rows
    u = rng.random(rows).astype(np.float32)
    out.append(dict(name="fp32_drafted_sparse", V=V, policies=pols,
                    arrays=dict(logits=x, uniforms=u, draft_tokens=draft,
                                cand_ids=cand, cand_probs=cp),
                    drafted_rows=rows - 1, kept_capacity=64))
    return out


def kwargs_of(case, J):
    kw = dict(case["arrays"])
    for k in ("histories", "generated", "mark_prompt", "kept_capacity", "drafted_rows"):
        if case.get(k) is not None:
            kw[k] = case[k]
    if case.get("stop"):
        kw["stop"] = tuple(case["stop"])
    return kw


def main():
    import jf_sampler as J
    import harness
    meta, arrays = [], {}
    for c in cases():
        pols = [J.policy(**p) for p in c["policies"]]
        res = harness.run_oracle(c["V"], pols, **kwargs_of(c, J))
        m = {k: v for k, v in c.items() if k != "arrays"}
        m["histories"] = None if c.get("histories") is None else [
            None if h is None else h.tolist() for h in c["histories"]]
        meta.append(m)
        for k, v in c["arrays"].items():
            arrays[f"{c['name']}/in/{k}"] = v
        for k, v in res.items():
            arrays[f"{c['name']}/out/{k}"] = v
    json.dump(meta, open(os.path.join(HERE, "select_cases.json"), "w"), indent=1)
    np.savez_compressed(os.path.join(HERE, "select_cases.npz"), **arrays)
    print("wrote", len(meta), "cases")


if __name__ == "__main__":
    main()
