"""GPU parity of jf_draft_select (the draft selector, through the C ABI)
against the CPU oracle: candidates, unary scores, proposed tokens and
proposal probabilities bit-exact (the oracle restates the same top-16 order,
edge-sum order and walk)."""
import numpy as np
import pytest

import jf_sampler as J
import oracle as O
from jf_sampler import workloads as WL

pytestmark = pytest.mark.gpu


def run_both(c, stride=None):
    import torch
    dev = torch.device("cuda", 0)
    lanes, V = c["lanes"], c["V"]
    print(f"draft case V={V} lanes={lanes} stride={stride}", flush=True)
    logits = c["logits"]
    if stride is not None:
        padded = np.zeros((logits.shape[0], stride), np.float32)
        padded[:, :V] = logits
        lg = torch.from_numpy(padded).to(dev)
    else:
        lg = torch.from_numpy(np.ascontiguousarray(logits)).to(dev)
    t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    hidden, pred, succ = t16(c["hidden"]), t16(c["pred"]), t16(c["succ"])
    u = torch.from_numpy(c["uniforms"]).to(dev)
    cand = torch.zeros((lanes * 7, 16), dtype=torch.int32, device=dev)
    unary = torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev)
    tokens = torch.zeros(lanes * 7, dtype=torch.int32, device=dev)
    q = torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev)
    sel = J.DraftSelector(V, lanes)
    pols = [J.policy(temperature=t) for t in c["temperatures"]]
    a = sel.args(logits=lg, hidden=hidden, pred_codebook=pred, succ_codebook=succ,
                 anchors=c["anchors"], policies=pols, candidates=cand, unary=unary,
                 tokens=tokens, q=q, uniforms=u, stride=stride)
    for _ in range(2):  # twice: the arrival counters return to zero
        sel.launch(a)
    torch.cuda.synchronize()
    g = dict(cand=cand.cpu().numpy().view(np.uint32).reshape(lanes, 7, 16),
             unary=unary.cpu().numpy().reshape(lanes, 7, 16),
             tokens=tokens.cpu().numpy().view(np.uint32).reshape(lanes, 7),
             q=q.cpu().numpy().reshape(lanes, 7, 16))
    sampled = [t > 0 for t in c["temperatures"]]
    rc, ru, rt, rq = O.draft_select(logits, c["hidden"], c["pred"], c["succ"], c["anchors"],
                                    c["temperatures"], sampled, c["uniforms"])
    sel.close()
    return g, dict(cand=rc, unary=ru, tokens=rt, q=rq), sampled


def assert_same(g, r, sampled):
    assert np.array_equal(g["cand"], r["cand"])
    assert np.array_equal(g["unary"].view(np.uint32), r["unary"].view(np.uint32))
    assert np.array_equal(g["tokens"], r["tokens"])
    for l, s in enumerate(sampled):
        if s:
            assert np.array_equal(g["q"][l].view(np.uint32), r["q"][l].view(np.uint32))


def test_draft_select_full_vocabulary():
    c = WL.config_draft()
    g, r, sampled = run_both(c)
    assert_same(g, r, sampled)


# 8192 * 40 + 3: 41 chunks, past the 32 one half-wave of list heads holds.
@pytest.mark.parametrize("V,stride", [(3000, None), (8192 * 2 + 5, 8192 * 2 + 7), (40000, None),
                                      (8192 * 40 + 3, None)])
def test_draft_select_shapes_ties_and_edge_rows(V, stride):
    c = WL.config_draft(V=V, lanes=3, seed=V)
    x = c["logits"]
    x[1] = np.round(x[1], 0)              # ties everywhere
    x[2] = 1.0                            # one value: the chunks' tie path
    x[3, ::2] = np.nan                    # NaN never enters
    x[4] = -np.inf
    x[4, [7, V - 1]] = [2.0, -3.0]        # fewer than 16 finite
    x[5] = np.nan
    x[5, :5] = [0.0, -0.0, 1.0, -0.0, 0.0]  # fewer than 16 non-NaN, signed zeros
    # About 100 equal largest tokens a chunk: more than 64 at or above the
    # chunk's bound, so the block's compaction ranks them.
    pick = np.random.default_rng(V + 1)
    for c0 in range(0, V, 8192):
        span = min(8192, V - c0)
        x[6, c0 + pick.choice(span, min(100, span), replace=False)] = 5.0
    c["anchors"][1] = 0xFFFFFFF0          # clamped into the codebooks
    c["temperatures"] = [0.0, 1.0, 0.3]
    g, r, sampled = run_both(c, stride)
    assert_same(g, r, sampled)
    assert g["cand"][0, 4, 15] == 0xFFFFFFFF  # query row 5: five non-NaN tokens


def test_edge_tables_feed_the_tree_builder():
    """The selector's edge tables (optional output) are bit-exact against the
    oracle's edge sums, and the host tree builder over the GPU's candidates,
    unary scores and tables equals the oracle's tree (greedy lanes, and
    sampled lanes with their walk as the forced chain)."""
    import torch
    c = WL.config_draft(V=40000, lanes=3, seed=9)
    c["temperatures"] = [0.0, 0.9, 0.0]
    lanes, V = c["lanes"], c["V"]
    dev = torch.device("cuda", 0)
    t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    lg = torch.from_numpy(c["logits"]).to(dev)
    cand = torch.zeros((lanes * 7, 16), dtype=torch.int32, device=dev)
    unary = torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev)
    tokens = torch.zeros(lanes * 7, dtype=torch.int32, device=dev)
    q = torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev)
    tables = torch.zeros((lanes, 7, 16, 16), dtype=torch.float32, device=dev)
    sel = J.DraftSelector(V, lanes)
    a = sel.args(logits=lg, hidden=t16(c["hidden"]), pred_codebook=t16(c["pred"]),
                 succ_codebook=t16(c["succ"]), anchors=c["anchors"],
                 policies=[J.policy(temperature=t) for t in c["temperatures"]],
                 candidates=cand, unary=unary, tokens=tokens, q=q,
                 uniforms=torch.from_numpy(c["uniforms"]).to(dev), edge_tables=tables)
    sel.launch(a)
    torch.cuda.synchronize()
    g_cand = cand.cpu().numpy().view(np.uint32).reshape(lanes, 7, 16)
    g_un = unary.cpu().numpy().reshape(lanes, 7, 16)
    g_tok = tokens.cpu().numpy().view(np.uint32).reshape(lanes, 7)
    g_tab = tables.cpu().numpy()
    sel.close()
    sampled = [t > 0 for t in c["temperatures"]]
    rc, ru, rt, _ = O.draft_select(c["logits"], c["hidden"], c["pred"], c["succ"], c["anchors"],
                                   c["temperatures"], sampled, c["uniforms"])
    assert np.array_equal(g_cand, rc) and np.array_equal(g_tok, rt)
    for l in range(lanes):
        want = np.zeros((7, 16, 16), np.float32)
        for p in range(7):
            h = c["hidden"][l * 8 + p + 1]
            for i in range(16 if p else 1):
                pid = min(int(rc[l, p - 1, i]) if p else int(c["anchors"][l]), V - 1)
                for j in range(16):
                    want[p, i, j] = O.draft_edge(c["pred"][pid], h, c["succ"][min(int(rc[l, p, j]), V - 1)])
        got = g_tab[l].copy()
        got[0, 1:] = 0.0  # position 0 has the anchor's row only
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        picks = None
        if sampled[l]:
            picks = np.array([int(np.nonzero(rc[l, p] == rt[l, p])[0][0]) for p in range(7)], np.uint32)
        tree = J.build_draft_tree(g_cand[l], g_un[l], got, int(c["anchors"][l]), 16, picks)
        ref = O.build_draft_tree(rc[l], ru[l], want, int(c["anchors"][l]), 16, picks)
        for k in ("rows", "copies", "parent", "depth", "copy", "token", "path_length", "path"):
            assert tree[k] == ref[k], (l, k)
