"""Runs one selection through the C ABI (HIP) and through the CPU oracle on the
same host inputs, so tests compare the two result dicts field by field."""
import numpy as np

import jf_sampler as J
import oracle as O

NO = 0xFFFFFFFF


def _policy_tuple(p):
    return (p.top_k, p.temperature, p.top_p, p.min_p, p.repetition, p.presence,
            p.frequency, p.flags)


def run_gpu(V, policies, *, logits=None, logits_bf16=None, masks=None,
            histories=None, generated=None, pending=None, mark_prompt=None,
            extra=None, uniforms=None, draft_tokens=None, drafted_rows=None,
            cand_ids=None, cand_probs=None, dense_q=None, stop=(NO, NO),
            kept_capacity=0, sampler=None, repeat=1):
    """Inputs are host numpy arrays with one row per selected row."""
    import torch
    dev = torch.device("cuda", 0)
    rows = len(policies)
    if logits is not None:
        lg = torch.from_numpy(np.ascontiguousarray(logits, np.float32)).to(dev)
    else:
        lg = torch.from_numpy(np.ascontiguousarray(logits_bf16, np.uint16).view(np.int16)).to(dev).view(torch.bfloat16)
    s = sampler or J.Sampler(V, max(rows, 1))
    kw = {}
    if masks is not None:
        kw["masks"] = torch.from_numpy(np.ascontiguousarray(masks, np.uint32).view(np.int32)).to(dev)
    table = None
    if histories is not None:
        H = max((len(h) for h in histories if h is not None), default=0) + 8
        table = J.PenaltyTable(V, rows, H + 32)
        for r, h in enumerate(histories):
            if h is None:
                continue
            table.rebuild(r, h, generated[r], None if pending is None else pending[r],
                          bool(mark_prompt[r]) if mark_prompt is not None else False)
        kw["penalties"] = table
        kw["penalty_rows"] = list(range(rows))
    if extra is not None:
        width = max(1, max(len(e) for e in extra))
        ex = np.zeros((rows, width), np.uint32)
        for r, e in enumerate(extra):
            ex[r, :len(e)] = e
        kw["extra_tokens"] = torch.from_numpy(ex.view(np.int32)).to(dev)
        kw["extra_counts"] = [len(e) for e in extra]
        kw["extra_stride"] = width
    if uniforms is not None:
        kw["uniforms"] = torch.from_numpy(np.ascontiguousarray(uniforms, np.float32)).to(dev)
    if draft_tokens is not None:
        kw["draft_tokens"] = torch.from_numpy(np.ascontiguousarray(draft_tokens, np.uint32).view(np.int32)).to(dev)
        kw["drafted_rows"] = rows if drafted_rows is None else drafted_rows
        if dense_q is not None:
            kw["dense_q"] = torch.from_numpy(np.ascontiguousarray(dense_q, np.float32)).to(dev)
        else:
            kw["cand_ids"] = torch.from_numpy(np.ascontiguousarray(cand_ids, np.uint32).view(np.int32)).to(dev)
            kw["cand_probs"] = torch.from_numpy(np.ascontiguousarray(cand_probs, np.float32)).to(dev)
    out = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    dp = torch.full((rows,), -7.0, dtype=torch.float32, device=dev)
    kept = None
    if kept_capacity:
        kept = (torch.zeros(rows, dtype=torch.int32, device=dev),
                torch.zeros((rows, kept_capacity), dtype=torch.int32, device=dev),
                torch.zeros((rows, kept_capacity), dtype=torch.float32, device=dev))
    for _ in range(repeat):
        s.sample(lg, policies, out, stop_tokens=stop, out_draft_probs=dp,
                 kept=kept, **kw)
    torch.cuda.synchronize()
    res = dict(tokens=out.cpu().numpy().view(np.uint32).copy(),
               draft_probs=dp.cpu().numpy().copy())
    if kept is not None:
        res["kept_counts"] = kept[0].cpu().numpy().view(np.uint32).copy()
        res["kept_ids"] = kept[1].cpu().numpy().view(np.uint32).copy()
        res["kept_probs"] = kept[2].cpu().numpy().copy()
    if table is not None:
        table.close()
    return res


def run_oracle(V, policies, *, logits=None, logits_bf16=None, masks=None,
               histories=None, generated=None, pending=None, mark_prompt=None,
               extra=None, uniforms=None, draft_tokens=None, drafted_rows=None,
               cand_ids=None, cand_probs=None, dense_q=None, stop=(NO, NO),
               kept_capacity=0, **_):
    rows = len(policies)
    toks = np.zeros(rows, np.uint32)
    dps = np.zeros(rows, np.float32)
    kc = np.zeros(rows, np.uint32)
    kid = np.zeros((rows, max(kept_capacity, 1)), np.uint32)
    kpr = np.zeros((rows, max(kept_capacity, 1)), np.float32)
    for r in range(rows):
        p = O.policy_from(policies[r])
        words = None
        if histories is not None and histories[r] is not None:
            rc, words = O.rebuild_penalty_words(
                V, histories[r], generated[r], None if pending is None else pending[r],
                bool(mark_prompt[r]) if mark_prompt is not None else False)
            assert rc == 0
        drafted = draft_tokens is not None and r < (rows if drafted_rows is None else drafted_rows)
        d = int(draft_tokens[r]) if drafted else NO
        t, dp, n, M, ids, probs = O.select_row(
            V, p,
            logits=None if logits is None else logits[r],
            logits_bf16=None if logits_bf16 is None else logits_bf16[r],
            mask=None if masks is None else masks[r], words=words,
            extra=None if extra is None else extra[r],
            uniform=0.0 if uniforms is None else float(uniforms[r]),
            draft_token=d,
            cand_ids=None if (cand_ids is None or not drafted) else cand_ids[r],
            cand_probs=None if (cand_probs is None or not drafted) else cand_probs[r],
            dense_q=None if (dense_q is None or not drafted) else dense_q[r],
            stop=stop, kept_capacity=kept_capacity)
        toks[r], dps[r], kc[r] = t, dp, n
        if kept_capacity:
            kid[r, :len(ids)] = ids
            kpr[r, :len(probs)] = probs
    res = dict(tokens=toks, draft_probs=dps)
    if kept_capacity:
        res["kept_counts"] = kc
        res["kept_ids"] = kid
        res["kept_probs"] = kpr
    return res


def assert_same(gpu, ref, *, check_draft=True, sampled_rows=None):
    """Bit-exact equality of tokens, draft probabilities and kept sets."""
    np.testing.assert_array_equal(gpu["tokens"], ref["tokens"])
    if check_draft:
        rows = sampled_rows if sampled_rows is not None else slice(None)
        np.testing.assert_array_equal(gpu["draft_probs"][rows], ref["draft_probs"][rows])
    if "kept_counts" in ref:
        np.testing.assert_array_equal(gpu["kept_counts"], ref["kept_counts"])
        cap = ref["kept_ids"].shape[1]
        for r in range(len(ref["tokens"])):
            n = min(int(ref["kept_counts"][r]), cap)
            np.testing.assert_array_equal(gpu["kept_ids"][r, :n], ref["kept_ids"][r, :n])
            np.testing.assert_array_equal(gpu["kept_probs"][r, :n], ref["kept_probs"][r, :n])
