"""Counted tokens applied to the device penalty table in place
(jf_penalty_table_count / _count_rows, penalty_count_kernel): after a rebuild
and a sequence of counts (tokens already held, new tokens, one row many
times, more tokens than one launch carries, a row pushed past its chunk's
fixed slots), penalized selection through both select kernels (the fast
one reads the fixed slots, the general one the sorted entries and bucket
offsets) equals the oracle over the dense words that countPenaltyTokens
(Sampling.cpp:75-80) would hold."""
import numpy as np
import pytest

import jf_sampler as J
import oracle as O

pytestmark = pytest.mark.gpu

V = 151936


def _logits(rows, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)


def _select(table, words, lg, policies, uniforms, extra=None):
    """Selection on the GPU (through `table`) and in the oracle (through the
    dense `words`); extra tokens route the launch to the general kernel."""
    import torch
    dev = torch.device("cuda", 0)
    rows = lg.shape[0]
    s = J.Sampler(V, rows)
    out = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    kw = {}
    if extra is not None:
        ex = np.zeros((rows, 1), np.uint32)
        ex[:, 0] = extra
        kw = dict(extra_tokens=torch.from_numpy(ex.view(np.int32)).to(dev),
                  extra_counts=[1] * rows, extra_stride=1)
    s.sample(torch.from_numpy(lg).to(dev), policies, out, penalties=table,
             penalty_rows=list(range(rows)),
             uniforms=torch.from_numpy(uniforms).to(dev), **kw)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint32).copy()
    want = np.array([O.select_row(V, O.policy_from(policies[r]), logits=lg[r], words=words[r],
                                  extra=None if extra is None else [int(extra[r])],
                                  uniform=float(uniforms[r]))[0] for r in range(rows)], np.uint32)
    return got, want


@pytest.mark.parametrize("general", [False, True])
def test_counts_update_the_table_in_place(general):
    rows = 4
    rng = np.random.default_rng(7)
    histories = [rng.integers(0, V, 1500, dtype=np.uint32) for _ in range(rows)]
    generated = [700, 0, 1499, 10]
    table = J.PenaltyTable(V, rows, 4096)
    words = np.zeros((rows, V), np.uint32)
    for r in range(rows):
        table.rebuild(r, histories[r], generated[r], None, r % 2 == 0)
        rc, words[r] = O.rebuild_penalty_words(V, histories[r], generated[r], None, r % 2 == 0)
        assert rc == 0
    # Tokens already held, new ones, repeats, and one row many times: 150
    # pairs (one launch reading host-mapped updates).
    pr, pt = [], []
    for k in range(150):
        r = int(rng.integers(0, rows)) if k % 5 else 2
        if k % 3 == 0:
            t = int(histories[r][rng.integers(0, len(histories[r]))])
        elif k % 3 == 1:
            t = int(rng.integers(0, V))
        else:
            t = int(rng.integers(8192 * 3, 8192 * 3 + 50))  # one chunk, many repeats
        pr.append(r)
        pt.append(t)
    table.count_rows(pr, pt)
    table.count(1, pt[:40])  # the single-row entry point, in order
    for r, t in zip(pr, pt):
        words[r, t] += 1
    for t in pt[:40]:
        words[1, t] += 1
    pols = [J.policy(repetition=1.3, presence=0.6, frequency=0.4),
            J.policy(temperature=0.8, top_k=40, presence=1.5, frequency=1.0),
            J.policy(temperature=1.1, top_p=0.9, repetition=1.8),
            J.policy(temperature=0.6, min_p=0.05, top_k=200, frequency=2.0, repetition=0.7)]
    uniforms = rng.random(rows, dtype=np.float32)
    lg = _logits(rows, 11)
    # Penalized tokens near the top, so the counts decide the selections.
    for r in range(rows):
        lg[r, pt[r::rows]] += 6.0
    extra = rng.integers(0, V, rows).astype(np.uint32) if general else None
    got, want = _select(table, words, lg, pols, uniforms, extra)
    np.testing.assert_array_equal(got, want)
    table.close()


def test_row_pushed_past_its_slots_still_selects_exactly():
    """Counts that overflow one chunk's fixed slots take the row off the fast
    kernel; a later rebuild that fits puts it back."""
    rows = 2
    rng = np.random.default_rng(3)
    table = J.PenaltyTable(V, rows, 4096)
    words = np.zeros((rows, V), np.uint32)
    hist = [np.arange(0, 200, dtype=np.uint32), rng.integers(0, V, 900, dtype=np.uint32)]
    for r in range(rows):
        table.rebuild(r, hist[r], 100, None, True)
        words[r] = O.rebuild_penalty_words(V, hist[r], 100, None, True)[1]
    # 400 new tokens in chunk 0 of row 0: more than its 256 slots.
    new = np.arange(200, 600, dtype=np.uint32)
    table.count_rows([0] * len(new), new)
    words[0, new] += 1
    pols = [J.policy(repetition=1.5, presence=1.0), J.policy(temperature=0.9, top_k=30, frequency=1.2)]
    lg = _logits(rows, 5)
    lg[0, :600] += 5.0
    uniforms = rng.random(rows, dtype=np.float32)
    got, want = _select(table, words, lg, pols, uniforms)
    np.testing.assert_array_equal(got, want)
    for r in range(rows):
        table.rebuild(r, hist[r], 100, None, True)
        words[r] = O.rebuild_penalty_words(V, hist[r], 100, None, True)[1]
    got, want = _select(table, words, lg, pols, uniforms)
    np.testing.assert_array_equal(got, want)
    table.close()


def test_slots_widen_for_a_clustered_row():
    """A table laid out 256 slots to a chunk widens to 512 when a rebuilt row
    holds more than 256 ids in one chunk and 512 suffice: every fitting row
    is laid out again. Counts then update the wider layout in place, and a
    row pushed past 512 leaves the fast kernel. Selections bit-exact
    against the oracle at each stage."""
    rows = 3
    rng = np.random.default_rng(17)
    table = J.PenaltyTable(V, rows, 2048)  # 2048 * 1.5 <= 19 chunks * 256: 256 slots
    words = np.zeros((rows, V), np.uint32)
    hist = [rng.integers(0, V, 900, dtype=np.uint32),
            np.concatenate([np.arange(0, 300, dtype=np.uint32),
                            rng.integers(8192, V, 200, dtype=np.uint32)]),
            rng.integers(0, V, 700, dtype=np.uint32)]
    for r in (0, 2, 1):  # the clustered row last: the others are laid out again
        table.rebuild(r, hist[r], 100, None, True)
        words[r] = O.rebuild_penalty_words(V, hist[r], 100, None, True)[1]
    pols = [J.policy(repetition=1.4, presence=0.7),
            J.policy(temperature=0.9, top_k=30, frequency=1.2, presence=0.5),
            J.policy(temperature=1.0, top_p=0.8, repetition=1.6)]
    lg = _logits(rows, 23)
    lg[:, :700] += 4.0
    uniforms = rng.random(rows, dtype=np.float32)
    got, want = _select(table, words, lg, pols, uniforms)
    np.testing.assert_array_equal(got, want)
    # 150 new ids in row 1's first chunk (450 <= 512) and counts elsewhere.
    pr = [1] * 150 + [0, 2, 0, 2]
    pt = list(range(300, 450)) + [5, 6, 7, 8192 * 4 + 1]
    table.count_rows(pr, pt)
    for r, t in zip(pr, pt):
        words[r, t] += 1
    got, want = _select(table, words, lg, pols, uniforms)
    np.testing.assert_array_equal(got, want)
    # 100 more (550 > 512): row 1 takes select_kernel.
    more = list(range(450, 550))
    table.count_rows([1] * len(more), more)
    words[1, more] += 1
    got, want = _select(table, words, lg, pols, uniforms)
    np.testing.assert_array_equal(got, want)
    table.close()


def test_one_row_counted_past_one_argument_batch():
    """jf_penalty_table_count of 200 tokens on one row (more than one
    kernel-argument batch of 64: one launch reading host-mapped updates,
    one block applying them in order), repeated and new ids mixed, six such
    calls back to back on one table (more calls than the table's four
    mapped buffers, so later calls reuse buffers earlier launches read);
    penalized selections bit-exact against the oracle."""
    rows = 2
    rng = np.random.default_rng(29)
    table = J.PenaltyTable(V, rows, 4096)
    words = np.zeros((rows, V), np.uint32)
    hist = [rng.integers(0, V, 700, dtype=np.uint32), rng.integers(0, V, 300, dtype=np.uint32)]
    for r in range(rows):
        table.rebuild(r, hist[r], 50, None, r == 0)
        words[r] = O.rebuild_penalty_words(V, hist[r], 50, None, r == 0)[1]
    for call in range(6):
        r = call % rows
        toks = np.concatenate([hist[r][:60], rng.integers(0, V, 100, dtype=np.uint32),
                               np.full(40, 8192 * 5 + 3, np.uint32)])
        rng.shuffle(toks)
        table.count(r, toks)
        for t in toks:
            words[r, t] += 1
    pols = [J.policy(temperature=0.9, top_k=40, presence=0.8, frequency=0.6, repetition=1.3),
            J.policy(repetition=1.5, presence=0.4)]
    lg = _logits(rows, 31)
    lg[:, hist[0][:60]] += 5.0
    uniforms = rng.random(rows, dtype=np.float32)
    got, want = _select(table, words, lg, pols, uniforms)
    np.testing.assert_array_equal(got, want)
    table.close()


def test_count_errors_leave_the_row_unchanged():
    table = J.PenaltyTable(1000, 2, 8)
    table.rebuild(0, [1, 2, 3], 1, None, True)
    with pytest.raises(RuntimeError, match="outside the vocabulary"):
        table.count_rows([0, 0], [5, 1000])
    with pytest.raises(RuntimeError, match="no penalty table row"):
        table.count_rows([0, 2], [5, 6])
    with pytest.raises(RuntimeError, match="exceeds the table row"):
        table.count(0, [10, 11, 12, 13, 14, 15, 16])  # 3 held + 7 new > 8
    table.count(0, [10, 11, 12, 13, 14])  # exactly 8
    table.close()


@pytest.mark.parametrize("bf16", [False, True])
def test_launch_split_between_fast_and_general_select(bf16):
    """A history clustered in low token ids (as real text is) overflows its
    first chunk's fixed slots: that row takes select_kernel while the other
    rows of the same call stay on the fast kernel. Greedy, cut and uncut
    rows, penalized and not; tokens bit-exact against the oracle."""
    from harness import run_gpu, run_oracle
    from jf_sampler import workloads as WL
    rng = np.random.default_rng(41 + bf16)
    rows = 7
    x = (rng.standard_normal((rows, V)) * 2.0).astype(np.float32)
    hist = [rng.integers(0, V, 800).astype(np.uint32) for _ in range(rows)]
    # Rows 2 and 5: Zipf-like ids, about 600 distinct below 8192.
    for r in (2, 5):
        hist[r] = np.minimum(rng.zipf(1.2, 3000), 8191).astype(np.uint32)
        x[r, :200] += 4.0
    pols = [J.policy(temperature=0.8, top_k=50, top_p=0.9, presence=0.5),
            J.policy(repetition=1.2),
            J.policy(temperature=0.7, top_k=40, frequency=0.8, presence=0.3),
            J.policy(temperature=1.0, presence=0.4),
            J.policy(temperature=0.9, top_k=50, top_p=0.9, presence=0.5),
            J.policy(repetition=1.3, presence=0.2),
            J.policy(temperature=1.0)]
    u = rng.random(rows).astype(np.float32)
    kw = dict(histories=hist, generated=[400] * rows, mark_prompt=[True] * rows, uniforms=u)
    if bf16:
        kw["logits_bf16"] = WL.to_bf16_bits(x)
    else:
        kw["logits"] = x
    g = run_gpu(V, pols, **kw)
    r = run_oracle(V, pols, **kw)
    np.testing.assert_array_equal(g["tokens"], r["tokens"])
    assert np.all(g["tokens"] != 0xFFFFFFFF)
