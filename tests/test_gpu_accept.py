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
