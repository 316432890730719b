"""The calls bench.py times, checked at full size: bench.GpuStep and
bench.VerifyStep build the same device inputs, penalty tables and argument
records as the timed loop, and one of their steps is compared with the
oracle row by row (bit-exact tokens, and the draft probabilities where the
step writes them). C2 and C5 run as benchmarked, without kept outputs or
draft probabilities; C1, C3 and C4 greedy and sampled as the bench issues
them, C4's selection and then its tree acceptance (retained and accepted
counts, path rows, the accepted tokens), as two calls and as the step the
bench times (jf_sample_accept_tree); C2 also with histories clustered
in low ids (every row, and every fourth row), which widen the penalty
table's fixed slots from 256 to 512 a chunk, and through the general
kernels (rows one float past 16-byte alignment, top-k 3000: select_kernel,
merge_kernel, the multi-pass stages); and the penalized chain-verify
step (4 lanes x 16 rows, V = 248,320: extras, sparse drafts, then chain
acceptance)."""
import numpy as np
import pytest

import bench
from harness import NO, run_oracle
from jf_sampler import workloads as WL

pytestmark = pytest.mark.gpu


def _oracle_for(w):
    """The oracle's results for the inputs GpuStep puts on the device."""
    kw = {}
    if "logits" in w:
        kw["logits"] = w["logits"]
    else:
        kw["logits_bf16"] = w["logits_bf16"]
    if "histories" in w:
        kw.update(histories=w["histories"], generated=w["generated"],
                  mark_prompt=[w["mark_prompt"]] * w["rows"])
    if "masks" in w:
        kw["masks"] = w["masks"]
    u = w.get("uniforms")
    if u is not None:
        if u.ndim == 2:  # C4: row k * 16 + r draws slot 24 + r of request k
            per = w["rows"] // u.shape[0]
            u = np.array([u[k, 24 + r] for k in range(u.shape[0]) for r in range(per)],
                         np.float32)
        kw["uniforms"] = u
    if w.get("tree") is not None and w.get("sampled"):
        c = w["tree"]
        draft = np.full(w["rows"], NO, np.uint32)
        for k, parent in enumerate(c["trees"]):
            for r in range(WL.chain_length(parent) - 1):
                draft[k * 16 + r] = c["tokens"][k][r + 1]
        kw.update(draft_tokens=draft, dense_q=c["q"])
    return run_oracle(w["V"], w["policies"], **kw)


@pytest.mark.parametrize("cfg,mode,history", [
    (2, "auto", "uniform"), (5, "auto", "uniform"), (1, "auto", "uniform"),
    (3, "greedy", "uniform"), (3, "sampled", "uniform"), (4, "greedy", "uniform"),
    (4, "sampled", "uniform"), (2, "auto", "zipf"), (2, "auto", "mixed"),
    (2, "general", "uniform")])
def test_benchmarked_step_matches_oracle(cfg, mode, history):
    import torch
    w = bench.build_workload(cfg, mode, history)
    print(f"bench call: {w['name']}", flush=True)
    g = bench.GpuStep(w)
    for i in (0, len(g.kw) - 1):  # the first and last rotated copy
        g.out.fill_(-1)
        g.sampler.launch(g.kw[i][0])  # the step's selection
        torch.cuda.synchronize()
        got = g.out.cpu().numpy().view(np.uint32).copy()
        want = _oracle_for(w) if i == 0 else want
        np.testing.assert_array_equal(got, want["tokens"])
        assert np.all(got != NO)
        if g.accept is not None:
            _check_tree_acceptance(g, w, want)
            # The step as benchmarked: jf_sample_accept_tree (one launch for
            # greedy lanes), the same results.
            g.out.fill_(-1)
            g.step(i)
            torch.cuda.synchronize()
            _check_tree_acceptance(g, w, want, launch=False)
        if g.draft_probs is not None:
            c = w["tree"]
            drafted = np.array([r < WL.chain_length(c["trees"][k]) - 1
                                for k in range(len(c["trees"])) for r in range(16)])
            assert drafted.any()
            dp = g.draft_probs.cpu().numpy()
            np.testing.assert_array_equal(dp[drafted], want["draft_probs"][drafted])
    del g
    torch.cuda.empty_cache()


def _check_tree_acceptance(g, w, want, launch=True):
    """The rest of C4's step: jf_accept_tree over the selected tokens (or,
    launch False, the results the step left), against the oracle's walk of
    each request's tree."""
    import torch
    import oracle as O
    c = w["tree"]
    rq = len(c["trees"])
    per = w["rows"] // rq
    if launch:
        g.sampler.launch_accept(g.accept)
        torch.cuda.synchronize()
    tt = g.out.cpu().numpy().view(np.uint32).reshape(rq, per)
    ret = g.acc_out[0].cpu().numpy()
    acc = g.acc_out[1].cpu().numpy()
    path = g.acc_path.cpu().numpy().view(np.uint32)
    for k in range(rq):
        tree = g.acc_trees[k]
        sampled = bool(w.get("sampled"))
        wt, wr, wa, wp = O.accept_tree(
            c["trees"][k], c["tokens"][k], tree.chain_rows if sampled else 0,
            list(tree.chain_q)[:8] if sampled else None, 8, sampled,
            want["tokens"][k * per:(k + 1) * per],
            want["draft_probs"][k * per:(k + 1) * per] if sampled else None,
            c["uniforms"][k] if sampled else None)
        assert ret[k] == wr and acc[k] == wa, (k, ret[k], wr, acc[k], wa)
        np.testing.assert_array_equal(path[k], wp)
        np.testing.assert_array_equal(tt[k, :wr], wt[:wr])


def test_benchmarked_verify_step_matches_oracle():
    import torch
    import oracle as O
    c = WL.config_verify()
    g = bench.VerifyStep(c)
    V, lanes, rows = c["V"], c["lanes"], c["rows"]
    print(f"bench call: {g.w['name']}", flush=True)
    vt, vp, chains = bench_oracle_verify(c)
    for i in (0, len(g.kw) - 1):
        g.out.fill_(-1)
        g.sampler.launch(g.kw[i][0])
        torch.cuda.synchronize()
        np.testing.assert_array_equal(g.out.cpu().numpy().view(np.uint32), vt)
        dp = g.draft_probs.cpu().numpy()
        drafted = c["draft_index"] != NO
        np.testing.assert_array_equal(dp[drafted], vp[drafted])
        g.sampler.launch_accept(g.accept)
        torch.cuda.synchronize()
        tt = g.out.cpu().numpy().view(np.uint32).reshape(lanes, rows)
        ret, acc = g.retained.cpu().numpy(), g.accepted.cpu().numpy()
        for l, (wt, wr, wa) in enumerate(chains):
            assert ret[l] == wr and acc[l] == wa, (l, ret[l], wr, acc[l], wa)
            np.testing.assert_array_equal(tt[l, :wr], wt[:wr])
    assert max(a for _, _, a in chains) >= 1  # some proposals are accepted
    g.close()
    del g
    torch.cuda.empty_cache()


def bench_oracle_verify(c):
    """The oracle's verify step: every row's selection, then each lane's chain
    acceptance (the same calls as bench.verify_cpu_baseline)."""
    import oracle as O
    V, lanes, rows = c["V"], c["lanes"], c["rows"]
    pol = O.policy(**c["policy"])
    inp = c["inputs"]
    vt = np.zeros(lanes * rows, np.uint32)
    vp = np.zeros(lanes * rows, np.float32)
    for l in range(lanes):
        words = O.rebuild_penalty_words(V, c["histories"][l], c["generated"][l], None,
                                        c["mark_prompt"])[1]
        for r in range(rows):
            g = l * rows + r
            d = int(c["draft_index"][g])
            ci = int(c["cand_index"][g])
            vt[g], vp[g] = O.select_row(
                V, pol, logits=c["logits"][g], words=words,
                extra=inp[l * rows + 1:l * rows + 1 + r], uniform=float(c["uniforms"][l, 15]),
                draft_token=int(inp[d]) if d != NO else NO,
                cand_ids=c["cand_ids"][ci] if d != NO else None,
                cand_probs=c["cand_probs"][ci] if d != NO else None)[:2]
    chains = []
    P = rows - 1
    for l in range(lanes):
        chains.append(O.accept_chain(P, rows, True, inp[l * rows + 1:(l + 1) * rows],
                                     vt[l * rows:(l + 1) * rows],
                                     cand_ids=c["cand_ids"][l * P:(l + 1) * P],
                                     cand_probs=c["cand_probs"][l * P:(l + 1) * P],
                                     target_draft_prob=vp[l * rows:(l + 1) * rows],
                                     uniforms40=c["uniforms"][l]))
    return vt, vp, chains


def test_cpp_loops_issue_the_draft_and_gather_calls():
    """bench.time_cpp_calls (libjf_bench_loop.so's draft and gather loops)
    issues the same calls as the Python wrappers: the draft selector's
    outputs after the loop equal one direct call's, and three in-place tree
    gathers from the loop leave the tensor as three direct calls do."""
    import torch
    import jf_sampler as J
    from gather_cases import gather_case
    dev = torch.device("cuda", 0)
    c = WL.config_draft(V=40000, lanes=3, seed=3)
    lanes, V = c["lanes"], c["V"]
    print(f"bench loops: draft V={V} lanes={lanes}, gather", flush=True)
    t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    x = torch.from_numpy(c["logits"]).to(dev)
    hidden, pred, succ = t16(c["hidden"]), t16(c["pred"]), t16(c["succ"])
    u = torch.from_numpy(c["uniforms"]).to(dev)
    outs = [torch.zeros((lanes * 7, 16), dtype=torch.int32, device=dev),
            torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev),
            torch.zeros(lanes * 7, dtype=torch.int32, device=dev),
            torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev)]
    sel = J.DraftSelector(V, lanes)
    pols = [J.policy(temperature=t) for t in c["temperatures"]]
    a = sel.args(logits=x, hidden=hidden, pred_codebook=pred, succ_codebook=succ,
                 anchors=c["anchors"], policies=pols, candidates=outs[0], unary=outs[1],
                 tokens=outs[2], q=outs[3], uniforms=u)
    # Rows the call leaves unwritten (a greedy lane's probabilities) keep
    # the fill in both runs.
    for o in outs:
        o.fill_(-1)
    sel.launch(a)
    torch.cuda.synchronize()
    want = [o.clone() for o in outs]
    for o in outs:
        o.fill_(-1)
    r = bench.time_cpp_calls("draft", [a], 4, batch=2, selector=sel)
    assert r["us_per_step"] > 0 and len(r["batch_us"]) == 2
    for o, w in zip(outs, want):
        assert torch.equal(o.view(torch.int32), w.view(torch.int32))
    sel.close()

    rng = np.random.default_rng(5)
    data, path, retained, p = gather_case(rng, lanes=6, layers=4, rows=16, columns=64,
                                          inner=64, pad=0)
    pr = torch.from_numpy(path.view(np.int32)).to(dev)
    rt = torch.from_numpy(retained.view(np.int32)).to(dev)
    direct = torch.from_numpy(data.view(np.int16)).to(dev)
    looped = direct.clone()
    ad = J.tree_gather_args(direct, pr, rt, **p)
    for _ in range(3):
        J.tree_gather(ad)
    bench.time_cpp_calls("gather", [J.tree_gather_args(looped, pr, rt, **p)], 3)
    torch.cuda.synchronize()
    assert torch.equal(direct, looped)
