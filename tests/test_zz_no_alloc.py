"""jf_sample_static (the entry point that allocates nothing, its scratch a
file-scope device array) against jf_sample on the same inputs: two calls in a
row, the second smaller, each bit-exact in tokens, draft probabilities and
kept outputs; then two all-greedy calls, the second smaller, which finish
through the array's packed chunk bests, and two calls of rows with no cut,
drawn in the select launch through the array's chunk summary words. Also
its size limits, which it rejects before any device call."""
import ctypes

import numpy as np
import pytest

import jf_sampler as J
from jf_sampler import workloads as WL

NO = 0xFFFFFFFF


def test_static_limits_are_rejected_before_any_device_call():
    a = J.JfSampleArgs()
    for V, rows, msg in ((0, 1, "geometry"), (262145, 1, "262144 tokens"),
                         (1000, 0, "1..64 rows"), (1000, 65, "1..64 rows")):
        a.rows = rows
        rc = J.lib().jf_sample_static(V, ctypes.byref(a), None)
        assert rc == J.JF_ERR_INVALID_ARGUMENT
        assert msg in J.lib().jf_last_error().decode()


def _case_inputs(which):
    """Host inputs: the headline C2 step, then a smaller mixed call."""
    if which == "c2":
        c = WL.config2()
        B = c["logits"].shape[0]
        return dict(V=c["V"], logits=c["logits"], policies=[J.policy(**c["policy"])] * B,
                    histories=c["histories"], generated=c["generated"],
                    uniforms=c["uniforms"], kept_capacity=64)
    if which in ("greedy", "greedy_small"):
        # Every row greedy: the selection finishes the rows itself through
        # the scratch's packed chunk bests, which each call leaves zeroed.
        rng = np.random.default_rng(78 if which == "greedy" else 79)
        V, rows = (151936, 24) if which == "greedy" else (20000, 3)
        x = rng.normal(0, 2, (rows, V)).astype(np.float32)
        x[0, [5, V - 1]] = 30.0  # the maximum in two chunks: the lower id
        histories = [rng.integers(0, V, 200).astype(np.uint32) if r % 3 == 1 else None
                     for r in range(rows)]
        pols = [J.policy(repetition=1.3, presence=0.4) if h is not None else J.policy()
                for h in histories]
        return dict(V=V, logits=x, policies=pols, histories=histories,
                    generated=[100] * rows, uniforms=rng.random(rows).astype(np.float32),
                    kept_capacity=0)
    if which in ("uncut", "uncut_small"):
        # Every row keeps every admitted token (no cut, draft, penalty or
        # kept output): each row's last chunk block draws it through the
        # array's chunk summary words, which each call returns to zero.
        rng = np.random.default_rng(80 if which == "uncut" else 81)
        V, rows = (151936, 16) if which == "uncut" else (20000, 3)
        x = rng.normal(0, 1.5, (rows, V)).astype(np.float32)
        pols = [J.policy(temperature=0.7 + 0.1 * (r % 5)) for r in range(rows)]
        return dict(V=V, logits=x, policies=pols, histories=None, generated=[0] * rows,
                    uniforms=rng.random(rows).astype(np.float32), kept_capacity=0)
    rng = np.random.default_rng(77)
    V, rows = 40000, 6
    x = np.round(rng.normal(0, 2, (rows, V)), 1).astype(np.float32)
    pols = [J.policy(), J.policy(temperature=0.8, top_k=40, top_p=0.9, presence=0.5),
            J.policy(temperature=1.0),  # no cut: the two-pass draw
            J.policy(temperature=0.6, min_p=0.1, top_k=300),
            J.policy(temperature=1.2, top_p=0.7, repetition=1.3),
            J.policy(temperature=0.9, top_k=5)]
    histories = [None if r in (0, 2, 5) else rng.integers(0, V, 300).astype(np.uint32)
                 for r in range(rows)]
    cand = rng.integers(0, V, (rows, 16)).astype(np.uint32)
    cand[:, 0] = np.argmax(x, axis=1)
    probs = rng.dirichlet(np.ones(16), rows).astype(np.float32)
    draft = cand[:, 0].copy()
    return dict(V=V, logits=x, policies=pols, histories=histories,
                generated=[100] * rows, uniforms=rng.random(rows).astype(np.float32),
                draft_tokens=draft, cand_ids=cand, cand_probs=probs, kept_capacity=0)


def _device_args(s, inp, dev):
    """JfSampleArgs for both entry points and their two sets of outputs."""
    import torch
    V, rows = inp["V"], len(inp["policies"])
    lg = torch.from_numpy(inp["logits"]).to(dev)
    kw, keep = {}, [lg]
    if inp.get("histories") is not None:
        H = max(len(h) for h in inp["histories"] if h is not None) + 8
        table = J.PenaltyTable(V, rows, H)
        for r, h in enumerate(inp["histories"]):
            if h is not None:
                table.rebuild(r, h, inp["generated"][r], None, False)
        kw["penalties"], kw["penalty_rows"] = table, list(range(rows))
        keep.append(table)
    kw["uniforms"] = torch.from_numpy(inp["uniforms"]).to(dev)
    if "draft_tokens" in inp:
        kw["draft_tokens"] = torch.from_numpy(inp["draft_tokens"].view(np.int32)).to(dev)
        kw["cand_ids"] = torch.from_numpy(inp["cand_ids"].view(np.int32)).to(dev)
        kw["cand_probs"] = torch.from_numpy(inp["cand_probs"]).to(dev)
    keep += list(kw.values())
    sets = []
    for _ in range(2):
        out = torch.full((rows,), -1, dtype=torch.int32, device=dev)
        dp = torch.full((rows,), -7.0, dtype=torch.float32, device=dev)
        kept = None
        cap = inp["kept_capacity"]
        if cap:
            kept = (torch.zeros(rows, dtype=torch.int32, device=dev),
                    torch.zeros((rows, cap), dtype=torch.int32, device=dev),
                    torch.zeros((rows, cap), dtype=torch.float32, device=dev))
        a, k = s.sample_args(lg, inp["policies"], out, out_draft_probs=dp, kept=kept, **kw)
        sets.append((a, k, out, dp, kept))
    return sets, keep


def _host(out, dp, kept):
    r = [out.cpu().numpy().view(np.uint32), dp.cpu().numpy()]
    if kept is not None:
        r += [kept[0].cpu().numpy(), kept[1].cpu().numpy(), kept[2].cpu().numpy()]
    return r


@pytest.mark.gpu
def test_static_entry_point_matches_jf_sample_on_two_calls():
    import torch
    dev = torch.device("cuda", 0)
    for which in ("c2", "small", "greedy", "greedy_small", "uncut", "uncut_small"):
        inp = _case_inputs(which)
        print(f"static vs sampler: case {which} V={inp['V']} rows={len(inp['policies'])}",
              flush=True)
        s = J.Sampler(inp["V"], len(inp["policies"]))
        sets, keep = _device_args(s, inp, dev)
        (a_ref, _, *ref), (a_sta, _, *sta) = sets
        s.launch(a_ref)
        J.sample_static(inp["V"], a_sta)
        torch.cuda.synchronize()
        want, got = _host(*ref), _host(*sta)
        for w, g in zip(want, got):
            np.testing.assert_array_equal(g, w)
        assert np.all(want[0] != NO)
        s.close()
