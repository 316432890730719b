"""GPU parity of chain and tree acceptance (jf_accept_chain / jf_accept_tree)
against the oracle, and the full C4 draft-tree verification: every tree row
selected (greedy argmax, or a draw with the chain rows' residual against the
dense draft q), then the tree walk. Accepted path lengths, paths and emitted
tokens must be bit-exact."""
import numpy as np
import pytest

import jf_sampler as J
import oracle as O
from jf_sampler import workloads as WL
from harness import NO, assert_same, run_gpu, run_oracle

pytestmark = pytest.mark.gpu


def tensor(a, dtype="i32"):
    import torch
    a = np.ascontiguousarray(a)
    if dtype == "i32":
        return torch.from_numpy(a.astype(np.uint32).view(np.int32)).cuda()
    return torch.from_numpy(a.astype(np.float32)).cuda()


def u32(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("VR", [8, 16])
def test_chain_acceptance(VR):
    import torch
    rng = np.random.default_rng(VR)
    lanes = 24
    P = VR - 1
    V = 1000
    target = rng.integers(0, 20, (lanes, VR)).astype(np.uint32)
    proposed = target[:, :P].copy()
    for l in range(lanes):  # diverge at a random position
        k = int(rng.integers(0, P + 1))
        if k < P:
            proposed[l, k] = (proposed[l, k] + 1) % 20
    proposed[5, 2] = NO
    cand = rng.integers(0, 20, (lanes, P, 16)).astype(np.uint32)
    cand[:, :, 3] = proposed
    cprob = rng.random((lanes, P, 16)).astype(np.float32)
    tprob = rng.random((lanes, VR)).astype(np.float32)
    uni = rng.random((lanes, 40)).astype(np.float32)
    maxret = [int(rng.integers(1, VR + 1)) for _ in range(lanes)]
    pols = [J.policy(temperature=0.7 if l % 2 else 0.0) for l in range(lanes)]
    stop = (13, NO)
    s = J.Sampler(V, lanes)
    tt = tensor(target)
    ret = torch.zeros(lanes, dtype=torch.int32, device="cuda")
    acc = torch.zeros(lanes, dtype=torch.int32, device="cuda")
    s.accept_chain(verify_rows=VR, proposed=tensor(proposed), target_tokens=tt,
                   retained=ret, accepted=acc, maximum_retained=maxret,
                   policies=pols, candidates=tensor(cand), proposal_probs=tensor(cprob, "f32"),
                   target_draft_probs=tensor(tprob, "f32"), uniforms=tensor(uni, "f32"),
                   stop_tokens=stop)
    torch.cuda.synchronize()
    for l in range(lanes):
        want_t, want_r, want_a = O.accept_chain(
            P, maxret[l], pols[l].temperature > 0, proposed[l], target[l], cand[l],
            cprob[l], tprob[l], uni[l], stop)
        assert u32(acc)[l] == want_a and u32(ret)[l] == want_r
        np.testing.assert_array_equal(u32(tt)[l], want_t)


def test_chain_acceptance_rejects_bad_limits():
    s = J.Sampler(100, 4)
    import torch
    z = torch.zeros(16, dtype=torch.int32, device="cuda")
    with pytest.raises(J.JfError) as e:
        s.accept_chain(verify_rows=8, proposed=z, target_tokens=z, retained=z,
                       accepted=z, maximum_retained=[9], policies=[J.policy()])
    assert "retention limit" in e.value.message
    with pytest.raises(J.JfError):
        s.accept_chain(verify_rows=12, proposed=z, target_tokens=z, retained=z,
                       accepted=z, maximum_retained=[1], policies=[J.policy()])


def c4_inputs(plant):
    c = WL.config4()
    rng = np.random.default_rng(44)
    requests, rows = len(c["trees"]), 16
    tokens = [t.copy() for t in c["tokens"]]
    if plant:
        # make some children carry the target argmax so greedy walks go deep
        am = c["logits"].argmax(axis=1).reshape(requests, rows)
        for q in range(requests):
            parent = c["trees"][q]
            for r in range(1, rows):
                if rng.random() < 0.6:
                    tokens[q][r] = am[q, parent[r]]
    return c, tokens


@pytest.mark.parametrize("plant", [False, True])
def test_c4_tree_greedy(plant):
    import torch
    c, tokens = c4_inputs(plant)
    V, requests, rows = c["V"], len(c["trees"]), 16
    pols = [J.policy()] * (requests * rows)
    g = run_gpu(V, pols, logits=c["logits"])
    r = run_oracle(V, pols, logits=c["logits"])
    assert_same(g, r, check_draft=False)
    s = J.Sampler(V, requests * rows)
    tt = tensor(g["tokens"].reshape(requests, rows))
    ret = torch.zeros(requests, dtype=torch.int32, device="cuda")
    acc = torch.zeros(requests, dtype=torch.int32, device="cuda")
    path = torch.zeros((requests, 8), dtype=torch.int32, device="cuda")
    trees = [J.tree_lane(c["trees"][q], tokens[q]) for q in range(requests)]
    s.accept_tree(trees=trees, rows_per_lane=rows, target_tokens=tt, retained=ret,
                  accepted=acc, path_rows=path, maximum_retained=[8] * requests,
                  policies=[J.policy()] * requests)
    torch.cuda.synchronize()
    depth = []
    for q in range(requests):
        want_t, want_r, want_a, want_p = O.accept_tree(
            c["trees"][q], tokens[q], 0, None, 8, False, r["tokens"][q * rows:(q + 1) * rows])
        assert u32(acc)[q] == want_a and u32(ret)[q] == want_r
        np.testing.assert_array_equal(u32(path)[q], want_p)
        np.testing.assert_array_equal(u32(tt)[q, :want_r], want_t[:want_r])
        depth.append(want_a)
    if plant:
        assert max(depth) >= 2


@pytest.mark.parametrize("plant", [False, True])
def test_c4_tree_sampled(plant):
    """Rejection-sampling acceptance along the tree: chain rows test u q < p
    and draw the residual max(p - q, 0) over the dense draft q; off-chain rows
    draw from the target with their own uniform 24 + row."""
    import torch
    c, tokens = c4_inputs(plant)
    V, requests, rows = c["V"], len(c["trees"]), 16
    q = c["q"]
    chain = [WL.chain_length(t) for t in c["trees"]]
    draft = np.full(requests * rows, NO, np.uint32)
    for k in range(requests):
        for r in range(chain[k] - 1):
            draft[k * rows + r] = tokens[k][r + 1]
    uidx = np.array([k * 40 + 24 + r for k in range(requests) for r in range(rows)], np.uint32)
    uflat = c["uniforms"].reshape(-1)
    pols = [J.policy(temperature=1.0)] * (requests * rows)
    kw = dict(logits=c["logits"], draft_tokens=draft, dense_q=q)
    import jf_sampler
    dev = torch.device("cuda", 0)
    s = J.Sampler(V, requests * rows)
    lg = torch.from_numpy(c["logits"]).to(dev)
    out = torch.zeros(requests * rows, dtype=torch.int32, device=dev)
    dp = torch.zeros(requests * rows, dtype=torch.float32, device=dev)
    s.sample(lg, pols, out, uniforms=tensor(uflat, "f32"), uniform_index=tensor(uidx),
             draft_tokens=tensor(draft), dense_q=torch.from_numpy(q).to(dev),
             out_draft_probs=dp)
    torch.cuda.synchronize()
    g = dict(tokens=u32(out).copy(), draft_probs=dp.cpu().numpy())
    r = run_oracle(V, pols, uniforms=uflat[uidx], **kw)
    assert_same(g, r)
    trees = []
    for k in range(requests):
        cq = [float(q[k * rows + j, tokens[k][j + 1]]) for j in range(chain[k] - 1)]
        trees.append(J.tree_lane(c["trees"][k], tokens[k], chain[k], cq))
    tt = tensor(g["tokens"].reshape(requests, rows))
    ret = torch.zeros(requests, dtype=torch.int32, device="cuda")
    acc = torch.zeros(requests, dtype=torch.int32, device="cuda")
    path = torch.zeros((requests, 8), dtype=torch.int32, device="cuda")
    s.accept_tree(trees=trees, rows_per_lane=rows, target_tokens=tt, retained=ret,
                  accepted=acc, path_rows=path, maximum_retained=[8] * requests,
                  policies=[J.policy(temperature=1.0)] * requests,
                  target_draft_probs=dp.reshape(requests, rows),
                  uniforms=tensor(c["uniforms"], "f32"))
    torch.cuda.synchronize()
    for k in range(requests):
        want_t, want_r, want_a, want_p = O.accept_tree(
            c["trees"][k], tokens[k], chain[k], list(trees[k].chain_q)[:8], 8, True,
            r["tokens"][k * rows:(k + 1) * rows], r["draft_probs"][k * rows:(k + 1) * rows],
            c["uniforms"][k])
        assert u32(acc)[k] == want_a and u32(ret)[k] == want_r
        np.testing.assert_array_equal(u32(path)[k], want_p)
        np.testing.assert_array_equal(u32(tt)[k, :want_r], want_t[:want_r])


def _random_trees(rng, lanes, R, argmax):
    """Trees of R rows in preorder (each parent an earlier row), their tokens
    planted with the parent row's argmax 60% of the time (greedy walks go
    deep), and the lanes' argmax rows."""
    trees, toks = [], []
    for q in range(lanes):
        parent = [NO] + [int(rng.integers(0, r)) for r in range(1, R)]
        tok = rng.integers(0, 1000, R).astype(np.uint32)
        for r in range(1, R):
            if rng.random() < 0.6:
                tok[r] = argmax[q * R + parent[r]]
        trees.append(parent)
        toks.append(tok)
    return trees, toks


@pytest.mark.parametrize("case", ["c4", "c4_planted", "r8_stops", "fallback_17_lanes"])
def test_sample_accept_tree_one_call(case):
    """jf_sample_accept_tree against jf_sample then jf_accept_tree on a second
    sampler: every row's token, each lane's retained and accepted counts and
    path rows equal. Greedy lanes over the selection's rows take one launch
    (each lane's last row finisher walks the tree); 17 lanes take the two
    calls. The full C4 tree step (16 lanes x 16 rows), with and without
    planted deep paths; 12 lanes x 8 rows with stop tokens on the paths."""
    import torch
    rng = np.random.default_rng(len(case))
    if case.startswith("c4"):
        c, tokens = c4_inputs(case == "c4_planted")
        V, R, lanes = c["V"], 16, len(c["trees"])
        x = c["logits"]
        trees = [J.tree_lane(c["trees"][q], tokens[q]) for q in range(lanes)]
        stops = (NO, NO)
    else:
        V = 151936
        R, lanes = 8, (12 if case == "r8_stops" else 17)
        x = rng.normal(0, 2.0, (lanes * R, V)).astype(np.float32)
        am = x.argmax(axis=1)
        par, toks = _random_trees(rng, lanes, R, am)
        trees = [J.tree_lane(par[q], toks[q]) for q in range(lanes)]
        stops = (int(am[3]), int(am[R + 1])) if case == "r8_stops" else (NO, NO)
    rows = lanes * R
    print(f"case {case}: {lanes} lanes x {R} rows, V={V}", flush=True)
    pols = [J.policy()] * rows
    lg = torch.from_numpy(x).cuda()
    results = []
    for combined in (True, False):
        s = J.Sampler(V, rows)
        out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
        ret = torch.full((lanes,), -1, dtype=torch.int32, device="cuda")
        acc = torch.full((lanes,), -1, dtype=torch.int32, device="cuda")
        path = torch.full((lanes, 8), -1, dtype=torch.int32, device="cuda")
        sa, keep_s = s.sample_args(lg, pols, out)
        ta, keep_t = s.accept_tree_args(
            trees=trees, rows_per_lane=R, target_tokens=out.view(lanes, R), retained=ret,
            accepted=acc, path_rows=path, maximum_retained=[8] * lanes,
            policies=[J.policy()] * lanes, stop_tokens=stops)
        for _ in range(2):  # twice: the words each call leaves are zero again
            if combined:
                s.launch_sample_accept_tree(sa, ta)
            else:
                s.launch(sa)
                s.launch_accept(("tree", ta, keep_t))
        torch.cuda.synchronize()
        results.append([u32(out).copy(), u32(ret).copy(), u32(acc).copy(), u32(path).copy()])
        s.close()
    for got, want in zip(*results):
        np.testing.assert_array_equal(got, want)
    # and the oracle's walk over the oracle's tokens
    want_tok = run_oracle(V, pols, logits=x)["tokens"]
    for q in range(lanes):
        par = list(trees[q].parent)[:trees[q].rows]
        tk = list(trees[q].token)[:trees[q].rows]
        wt, wr, wa, wp = O.accept_tree(par, tk, 0, None, 8, False,
                                       want_tok[q * R:(q + 1) * R], stop=stops)
        assert results[0][1][q] == wr and results[0][2][q] == wa, (q, wr, wa)
        np.testing.assert_array_equal(results[0][3][q], wp)
        np.testing.assert_array_equal(results[0][0][q * R:q * R + wr], wt[:wr])


def test_sample_accept_tree_expired_wait():
    """The combined call's bounded waits: with a bound of 0 every row's
    finisher gives up, the lanes' rows hold JF_NO_TOKEN and the status is
    reported once as JF_ERR_DEVICE; at the default bound the next calls are
    bit-exact again."""
    import torch
    c, tokens = c4_inputs(True)
    V, R, lanes = c["V"], 16, len(c["trees"])
    rows = lanes * R
    pols = [J.policy()] * rows
    lg = torch.from_numpy(c["logits"]).cuda()
    trees = [J.tree_lane(c["trees"][q], tokens[q]) for q in range(lanes)]
    s = J.Sampler(V, rows)
    out = torch.full((rows,), -1, dtype=torch.int32, device="cuda")
    ret = torch.zeros(lanes, dtype=torch.int32, device="cuda")
    acc = torch.zeros(lanes, dtype=torch.int32, device="cuda")
    path = torch.zeros((lanes, 8), dtype=torch.int32, device="cuda")
    sa, keep_s = s.sample_args(lg, pols, out)
    ta, keep_t = s.accept_tree_args(
        trees=trees, rows_per_lane=R, target_tokens=out.view(lanes, R), retained=ret,
        accepted=acc, path_rows=path, maximum_retained=[8] * lanes,
        policies=[J.policy()] * lanes)
    s.launch_sample_accept_tree(sa, ta)
    torch.cuda.synchronize()
    want = [u32(out).copy(), u32(ret).copy(), u32(acc).copy(), u32(path).copy()]
    s.set_wait_bound(0)
    s.launch_sample_accept_tree(sa, ta)
    torch.cuda.synchronize()
    assert np.all(u32(out) == NO)
    with pytest.raises(J.JfError) as e:
        s.status()
    assert e.value.code == J.JF_ERR_DEVICE
    s.set_wait_bound(1 << 20)
    for _ in range(2):
        s.launch_sample_accept_tree(sa, ta)
        torch.cuda.synchronize()
        for g, w in zip([u32(out), u32(ret), u32(acc), u32(path)], want):
            np.testing.assert_array_equal(g, w)
    s.status()
