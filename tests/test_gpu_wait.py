"""The finishers' bounded waits (no counterpart in the reference, whose
last-arriving group never waits; split_reduce.h:14-45): their expiry path,
driven from the host by a wait bound of 0, so that every kernel still exits
normally. Both finisher forms: the row's last chunk block (V = 151,936, 19
chunks) and the last block to arrive (V = 8,000, one chunk). Expiry gives
JF_NO_TOKEN rows and a status the host reports once as JF_ERR_DEVICE (by
jf_sampler_status, or by the next jf_sample before it enqueues anything);
the words the expired call left are cleared, and the next calls at the
default bound are bit-exact with the oracle again. The same for the draw of
rows with no cut finished in the select launch."""
import numpy as np
import pytest

import jf_sampler as J
from harness import NO, run_oracle

pytestmark = pytest.mark.gpu


def greedy_call(s, x):
    import torch
    dev = torch.device("cuda", 0)
    out = torch.full((x.shape[0],), -1, dtype=torch.int32, device=dev)
    s.sample(torch.from_numpy(x).to(dev), [J.policy()] * x.shape[0], out)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32).copy()


@pytest.mark.parametrize("V", [151936, 8000])
def test_expired_wait_reports_and_recovers(V):
    import torch
    print(f"case V={V}", flush=True)
    rng = np.random.default_rng(V)
    rows = 8
    x = rng.normal(0, 2.0, (rows, V)).astype(np.float32)
    want = run_oracle(V, [J.policy()] * rows, logits=x)["tokens"]
    s = J.Sampler(V, rows)
    np.testing.assert_array_equal(greedy_call(s, x), want)
    s.status()  # nothing to report

    # Bound 0: every row's finisher gives up.
    s.set_wait_bound(0)
    got = greedy_call(s, x)
    assert np.all(got == NO), got
    with pytest.raises(J.JfError) as e:
        s.status()
    assert e.value.code == J.JF_ERR_DEVICE and "expired" in e.value.message
    s.status()  # reported once
    s.set_wait_bound(1 << 20)
    np.testing.assert_array_equal(greedy_call(s, x), want)

    # The next jf_sample reports it instead, enqueuing nothing, then recovers.
    s.set_wait_bound(0)
    assert np.all(greedy_call(s, x) == NO)
    s.set_wait_bound(1 << 20)
    dev = torch.device("cuda", 0)
    out = torch.full((rows,), 7, dtype=torch.int32, device=dev)
    with pytest.raises(J.JfError) as e:
        s.sample(torch.from_numpy(x).to(dev), [J.policy()] * rows, out)
    assert e.value.code == J.JF_ERR_DEVICE
    torch.cuda.synchronize()
    assert np.all(out.cpu().numpy() == 7)  # nothing ran
    for _ in range(3):
        np.testing.assert_array_equal(greedy_call(s, x), want)
    s.status()


def test_expired_wait_of_the_in_launch_draw():
    """Rows with no cut drawn by each row's last chunk block (its gather of
    the other chunks' summary words is the same bounded wait): bound 0 gives
    JF_NO_TOKEN rows and one JF_ERR_DEVICE report; the next calls at the
    default bound are bit-exact again."""
    import torch
    V, rows = 5 * 8192 + 76, 6  # 16-byte aligned rows: the fast kernel's launch
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1.5, (rows, V)).astype(np.float32)
    u = rng.random(rows).astype(np.float32)
    pols = [J.policy(temperature=0.9)] * rows
    want = run_oracle(V, pols, logits=x, uniforms=u)["tokens"]
    dev = torch.device("cuda", 0)
    s = J.Sampler(V, rows)
    xt, ut = torch.from_numpy(x).to(dev), torch.from_numpy(u).to(dev)

    def call():
        out = torch.full((rows,), -1, dtype=torch.int32, device=dev)
        s.sample(xt, pols, out, uniforms=ut)
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.uint32).copy()

    np.testing.assert_array_equal(call(), want)
    s.set_wait_bound(0)
    assert np.all(call() == NO)
    with pytest.raises(J.JfError) as e:
        s.status()
    assert e.value.code == J.JF_ERR_DEVICE
    s.set_wait_bound(1 << 20)
    for _ in range(3):
        np.testing.assert_array_equal(call(), want)
    s.status()


def test_expired_wait_of_the_residual_draw():
    """Drafted rows with no cut drawn by the residual launch's finisher (each
    row's last chunk block gathers the other chunks' slice words, the same
    bounded wait), beside undrafted rows drawn in blocks of their own: bound
    0 gives the drafted rows JF_NO_TOKEN, the others their tokens, and one
    JF_ERR_DEVICE report; the next calls at the default bound are bit-exact
    again."""
    import torch
    V, rows, drafted = 5 * 8192 + 76, 6, 4
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1.5, (rows, V)).astype(np.float32)
    u = rng.random(rows).astype(np.float32)
    q = rng.dirichlet(np.ones(V) * 0.5, rows).astype(np.float32)
    d = rng.integers(0, V, rows).astype(np.uint32)
    pols = [J.policy(temperature=0.9)] * rows
    ref = run_oracle(V, pols, logits=x, uniforms=u, draft_tokens=d, drafted_rows=drafted,
                     dense_q=q)
    dev = torch.device("cuda", 0)
    s = J.Sampler(V, rows)
    xt, ut = torch.from_numpy(x).to(dev), torch.from_numpy(u).to(dev)
    dt = torch.from_numpy(d.view(np.int32)).to(dev)
    qt = torch.from_numpy(q).to(dev)

    def call():
        out = torch.full((rows,), -1, dtype=torch.int32, device=dev)
        dp = torch.full((rows,), -1.0, dtype=torch.float32, device=dev)
        s.sample(xt, pols, out, uniforms=ut, draft_tokens=dt, drafted_rows=drafted,
                 dense_q=qt, out_draft_probs=dp)
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.uint32).copy(), dp.cpu().numpy()

    def same(got):
        np.testing.assert_array_equal(got[0], ref["tokens"])
        np.testing.assert_array_equal(got[1], ref["draft_probs"])

    same(call())
    s.set_wait_bound(0)
    tokens, _ = call()
    assert np.all(tokens[:drafted] == NO), tokens
    np.testing.assert_array_equal(tokens[drafted:], ref["tokens"][drafted:])
    with pytest.raises(J.JfError) as e:
        s.status()
    assert e.value.code == J.JF_ERR_DEVICE
    s.set_wait_bound(1 << 20)
    for _ in range(3):
        same(call())
    s.status()
