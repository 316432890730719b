"""ctypes binding of the CPU oracle (oracle/_build/libjf_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline. The
product never imports it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libjf_oracle.so")
NO_TOKEN = 0xFFFFFFFF

c_u32, c_u64, c_f32, c_vp = ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float, ctypes.c_void_p


class Policy(ctypes.Structure):
    _fields_ = [("top_k", c_u32), ("temperature", c_f32), ("top_p", c_f32),
                ("min_p", c_f32), ("repetition", c_f32), ("presence", c_f32),
                ("frequency", c_f32), ("flags", c_u32)]


class RowInput(ctypes.Structure):
    _fields_ = [("logits", c_vp), ("logits_bf16", c_vp), ("mask", c_vp),
                ("words", c_vp), ("extra", c_vp), ("extra_count", c_u32),
                ("uniform", c_f32), ("draft_token", c_u32),
                ("cand_ids", c_vp), ("cand_probs", c_vp), ("dense_q", c_vp)]


class RowOutput(ctypes.Structure):
    _fields_ = [("token", c_u32), ("draft_probability", c_f32),
                ("kept_count", c_u32), ("maximum", c_f32)]


class ChainParams(ctypes.Structure):
    _fields_ = [("proposals", c_u32), ("remaining", c_u32), ("stop0", c_u32),
                ("stop1", c_u32), ("sampled", ctypes.c_int)]


class TreeParams(ctypes.Structure):
    _fields_ = [("rows", c_u32), ("chain_rows", c_u32), ("remaining", c_u32),
                ("stop0", c_u32), ("stop1", c_u32), ("sampled", ctypes.c_int),
                ("parent", c_u32 * 16), ("token", c_u32 * 16),
                ("chain_q", c_f32 * 8)]


class DraftLane(ctypes.Structure):
    _fields_ = [("vocabulary", c_u32), ("anchor", c_u32), ("temperature", c_f32),
                ("sampled", ctypes.c_int)]


class GatherParams(ctypes.Structure):
    _fields_ = [(n, c_u32) for n in ("columns", "inner", "inner_stride", "outer_stride",
                                     "row_stride", "lane_stride", "layer_stride", "layers",
                                     "lanes", "rows")]


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _bind(ctypes.CDLL(LIB_PATH))
    return _lib


def native_lib(directory):
    """The same source built with -O3 -march=native into `directory` (the CPU
    baseline's build, made on the machine that runs it)."""
    subprocess.run(["make", "-s", "-C", HERE, "native", f"NATIVE={directory}"], check=True)
    return _bind(ctypes.CDLL(os.path.join(directory, "libjf_oracle_native.so")))


def _bind(L):
    L.jfo_logit_key.argtypes = [c_f32]
    L.jfo_logit_key.restype = c_u32
    L.jfo_key_logit.argtypes = [c_u32]
    L.jfo_key_logit.restype = c_f32
    L.jfo_expf.argtypes = [c_f32]
    L.jfo_expf.restype = c_f32
    L.jfo_floor_mul.argtypes = [c_u64, c_f32]
    L.jfo_floor_mul.restype = c_u64
    L.jfo_residual.argtypes = [c_u64, c_u64, c_f32]
    L.jfo_residual.restype = c_u64
    L.jfo_exp64.argtypes = [ctypes.c_double]
    L.jfo_exp64.restype = ctypes.c_double
    L.jfo_chunk_scale.argtypes = [c_f32, c_f32, c_f32]
    L.jfo_chunk_scale.restype = c_u64
    L.jfo_scale_by.argtypes = [c_u64, c_u64]
    L.jfo_scale_by.restype = c_u64
    L.jfo_uncut_probability.argtypes = [c_f32, c_u64, c_u64]
    L.jfo_uncut_probability.restype = c_f32
    L.jfo_splitmix64.argtypes = [c_u64, c_u64]
    L.jfo_splitmix64.restype = c_u64
    L.jfo_next_uniform.argtypes = [c_u64, ctypes.POINTER(c_u64)]
    L.jfo_next_uniform.restype = c_f32
    L.jfo_stage_cycle.argtypes = [c_u64, ctypes.POINTER(c_u64), c_u32,
                                  ctypes.c_int, c_vp]
    L.jfo_stage_cycle.restype = None
    L.jfo_rebuild_penalty_words.argtypes = [
        c_vp, c_u32, c_vp, c_u64, c_u64, ctypes.c_int, c_u32, ctypes.c_int]
    L.jfo_count_penalty_tokens.argtypes = [c_vp, c_u32, c_vp, c_u64]
    L.jfo_penalize_logit.argtypes = [c_f32, c_u32, c_f32, c_f32, c_f32, c_f32]
    L.jfo_penalize_logit.restype = c_f32
    L.jfo_repetition_inverse.argtypes = [c_f32]
    L.jfo_repetition_inverse.restype = c_f32
    L.jfo_policy_valid.argtypes = [ctypes.POINTER(Policy)]
    L.jfo_select_row.argtypes = [c_u32, c_u32, c_u32, ctypes.POINTER(Policy),
                                 ctypes.POINTER(RowInput),
                                 ctypes.POINTER(RowOutput), c_vp, c_vp, c_u32]
    L.jfo_select_batch.argtypes = [
        c_u32, c_u32, c_u32, c_u32, ctypes.POINTER(Policy), c_vp,
        ctypes.c_int, c_u64, c_vp, c_u64, c_vp, c_vp, c_vp, c_vp, c_vp, c_u32]
    L.jfo_accept_chain.argtypes = [ctypes.POINTER(ChainParams), c_vp, c_vp,
                                   c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]
    L.jfo_accept_chain.restype = None
    L.jfo_accept_tree.argtypes = [ctypes.POINTER(TreeParams), c_vp, c_vp,
                                  c_vp, c_vp, c_vp, c_vp]
    L.jfo_accept_tree.restype = None
    L.jfo_draft_top16.argtypes = [c_vp, c_u32, c_vp, c_vp]
    L.jfo_draft_top16.restype = None
    L.jfo_draft_edge.argtypes = [c_vp, c_vp, c_vp]
    L.jfo_draft_edge.restype = c_f32
    L.jfo_draft_select_lane.argtypes = [ctypes.POINTER(DraftLane), c_vp, c_u64, c_vp,
                                        c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]
    L.jfo_draft_select_lane.restype = None
    L.jfo_tree_gather.argtypes = [c_vp, c_vp, c_vp, ctypes.POINTER(GatherParams)]
    L.jfo_tree_gather.restype = None
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(c_vp)


def policy(top_k=0, temperature=0.0, top_p=1.0, min_p=0.0, repetition=1.0,
           presence=0.0, frequency=0.0, constrained=False, exclude_stop=False):
    return Policy(top_k, temperature, top_p, min_p, repetition, presence,
                  frequency, (1 if constrained else 0) | (2 if exclude_stop else 0))


def policy_from(p):
    """An oracle Policy with the fields of a jf_sampler.JfPolicy."""
    return Policy(p.top_k, p.temperature, p.top_p, p.min_p, p.repetition,
                  p.presence, p.frequency, p.flags)


def select_row(vocabulary, pol, *, logits=None, logits_bf16=None, mask=None,
               words=None, extra=None, uniform=0.0, draft_token=NO_TOKEN,
               cand_ids=None, cand_probs=None, dense_q=None,
               stop=(NO_TOKEN, NO_TOKEN), kept_capacity=0):
    """One row: (token, draft_probability, kept_count, maximum, kept_ids,
    kept_probs)."""
    keep = []

    def arr(a, dt):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dt)
        keep.append(a)
        return a

    inp = RowInput()
    inp.logits = _p(arr(logits, np.float32))
    inp.logits_bf16 = _p(arr(logits_bf16, np.uint16))
    inp.mask = _p(arr(mask, np.uint32))
    inp.words = _p(arr(words, np.uint32))
    ex = arr(extra, np.uint32)
    inp.extra = _p(ex)
    inp.extra_count = 0 if ex is None else ex.size
    inp.uniform = uniform
    inp.draft_token = draft_token
    inp.cand_ids = _p(arr(cand_ids, np.uint32))
    inp.cand_probs = _p(arr(cand_probs, np.float32))
    inp.dense_q = _p(arr(dense_q, np.float32))
    out = RowOutput()
    kid = np.zeros(max(kept_capacity, 1), dtype=np.uint32)
    kpr = np.zeros(max(kept_capacity, 1), dtype=np.float32)
    rc = lib().jfo_select_row(vocabulary, stop[0], stop[1], ctypes.byref(pol),
                              ctypes.byref(inp), ctypes.byref(out),
                              _p(kid) if kept_capacity else None,
                              _p(kpr) if kept_capacity else None, kept_capacity)
    if rc:
        raise RuntimeError(f"oracle select_row failed: {rc}")
    n = min(out.kept_count, kept_capacity)
    return (out.token, out.draft_probability, out.kept_count, out.maximum,
            kid[:n].copy(), kpr[:n].copy())


def select_batch(vocabulary, policies, logits, *, is_bf16=False, masks=None,
                 words=None, pen_rows=None, uniforms=None,
                 stop=(NO_TOKEN, NO_TOKEN), threads=1, library=None):
    rows = logits.shape[0]
    pol = (Policy * rows)(*policies)
    out = np.zeros(rows, dtype=np.uint32)
    mx = np.zeros(rows, dtype=np.float32)
    rc = (library or lib()).jfo_select_batch(
        rows, vocabulary, stop[0], stop[1], pol, _p(logits), 1 if is_bf16 else 0,
        logits.shape[1], _p(masks), 0 if masks is None else masks.shape[1],
        _p(words), _p(pen_rows), _p(uniforms), _p(out), _p(mx), threads)
    if rc:
        raise RuntimeError(f"oracle select_batch failed: {rc}")
    return out, mx


def next_uniform(seed, counter):
    c = c_u64(counter)
    u = lib().jfo_next_uniform(seed, ctypes.byref(c))
    return u, c.value


def stage_cycle(seed, counter, verify_rows, tree_cycle):
    out = np.zeros(40, dtype=np.float32)
    c = c_u64(counter)
    lib().jfo_stage_cycle(seed, ctypes.byref(c), verify_rows,
                          1 if tree_cycle else 0, _p(out))
    return out, c.value


def rebuild_penalty_words(vocabulary, history, generated, pending=None,
                          mark_prompt=False):
    words = np.zeros(vocabulary, dtype=np.uint32)
    h = np.ascontiguousarray(history, dtype=np.uint32)
    rc = lib().jfo_rebuild_penalty_words(
        _p(words), vocabulary, _p(h), h.size, generated,
        0 if pending is None else 1, 0 if pending is None else pending,
        1 if mark_prompt else 0)
    return rc, words


def accept_chain(proposals, remaining, sampled, draft_tokens, target_tokens,
                 cand_ids=None, cand_probs=None, target_draft_prob=None,
                 uniforms40=None, stop=(NO_TOKEN, NO_TOKEN)):
    p = ChainParams(proposals, remaining, stop[0], stop[1], 1 if sampled else 0)
    tt = np.ascontiguousarray(target_tokens, dtype=np.uint32).copy()
    d = np.ascontiguousarray(draft_tokens, dtype=np.uint32)
    ci = None if cand_ids is None else np.ascontiguousarray(cand_ids, dtype=np.uint32)
    cp = None if cand_probs is None else np.ascontiguousarray(cand_probs, dtype=np.float32)
    tp = None if target_draft_prob is None else np.ascontiguousarray(target_draft_prob, dtype=np.float32)
    u = None if uniforms40 is None else np.ascontiguousarray(uniforms40, dtype=np.float32)
    ret, acc = c_u32(), c_u32()
    lib().jfo_accept_chain(ctypes.byref(p), _p(d), _p(ci), _p(cp), _p(tp),
                           _p(u), _p(tt), ctypes.byref(ret), ctypes.byref(acc))
    return tt, ret.value, acc.value


def accept_tree(parent, token, chain_rows, chain_q, remaining, sampled,
                target_tokens, target_draft_prob=None, uniforms40=None,
                stop=(NO_TOKEN, NO_TOKEN)):
    p = TreeParams()
    p.rows = len(parent)
    p.chain_rows = chain_rows
    p.remaining = remaining
    p.stop0, p.stop1 = stop
    p.sampled = 1 if sampled else 0
    for i, v in enumerate(parent):
        p.parent[i] = v
    for i, v in enumerate(token):
        p.token[i] = v
    for i, v in enumerate(chain_q or []):
        p.chain_q[i] = v
    tt = np.zeros(16, dtype=np.uint32)
    tt[:len(target_tokens)] = target_tokens
    tp = np.zeros(16, dtype=np.float32)
    if target_draft_prob is not None:
        tp[:len(target_draft_prob)] = target_draft_prob
    u = np.zeros(40, dtype=np.float32) if uniforms40 is None else np.ascontiguousarray(uniforms40, dtype=np.float32)
    ret, acc = c_u32(), c_u32()
    path = np.zeros(8, dtype=np.uint32)
    lib().jfo_accept_tree(ctypes.byref(p), _p(tp), _p(u), _p(tt),
                          ctypes.byref(ret), ctypes.byref(acc), _p(path))
    return tt, ret.value, acc.value, path


def draft_top16(row):
    """Exact top 16 of one fp32 row: (ids, values) in (value desc, id asc)."""
    r = np.ascontiguousarray(row, dtype=np.float32)
    ids = np.zeros(16, np.uint32)
    vals = np.zeros(16, np.float32)
    lib().jfo_draft_top16(_p(r), len(r), _p(ids), _p(vals))
    return ids, vals


def draft_edge(pred_row, hidden, succ_row):
    """One edge score over bf16 bit patterns (uint16 arrays of 256)."""
    a = [np.ascontiguousarray(x, dtype=np.uint16) for x in (pred_row, hidden, succ_row)]
    return lib().jfo_draft_edge(_p(a[0]), _p(a[1]), _p(a[2]))


def draft_select(logits, hidden, pred_codebook, succ_codebook, anchors, temperatures,
                 sampled, uniforms40):
    """Every lane of a draft selection: logits [lanes*8][V] fp32, hidden
    [lanes*8][256] bf16 bits, codebooks [V][256] bf16 bits, uniforms40
    [lanes][40]. Returns candidates, unary, tokens, q (q zero for greedy
    lanes)."""
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    hidden = np.ascontiguousarray(hidden, dtype=np.uint16)
    pc = np.ascontiguousarray(pred_codebook, dtype=np.uint16)
    sc = np.ascontiguousarray(succ_codebook, dtype=np.uint16)
    u = np.ascontiguousarray(uniforms40, dtype=np.float32)
    lanes = len(anchors)
    V = logits.shape[1]
    cand = np.zeros((lanes, 7, 16), np.uint32)
    unary = np.zeros((lanes, 7, 16), np.float32)
    tokens = np.zeros((lanes, 7), np.uint32)
    q = np.zeros((lanes, 7, 16), np.float32)
    for l in range(lanes):
        lane = DraftLane(V, int(anchors[l]), float(temperatures[l]), 1 if sampled[l] else 0)
        lg = np.ascontiguousarray(logits[l * 8:(l + 1) * 8])
        hd = np.ascontiguousarray(hidden[l * 8:(l + 1) * 8])
        c, un, t, qq = cand[l], unary[l], tokens[l], q[l]
        lib().jfo_draft_select_lane(ctypes.byref(lane), _p(lg), V, _p(hd), _p(pc), _p(sc),
                                    _p(np.ascontiguousarray(u[l])), _p(c), _p(un), _p(t), _p(qq))
    return cand, unary, tokens, q


def tree_gather(data, path_rows, retained, **params):
    """verify_tree_gather in place on a copy of `data` (uint16); returns it."""
    out = np.ascontiguousarray(data, dtype=np.uint16).copy()
    pr = np.ascontiguousarray(path_rows, dtype=np.uint32)
    rt = np.ascontiguousarray(retained, dtype=np.uint32)
    p = GatherParams(**params)
    lib().jfo_tree_gather(_p(out), _p(pr), _p(rt), ctypes.byref(p))
    return out


# ---- draft tree builder (Runtime.cpp:58-174), pure Python ------------------
#
# The frontier is Python's heapq ordered by (-logp, pick, insertion order).
# The reference's std::priority_queue breaks exact (logp, pick) ties by its
# heap layout instead; the tests use inputs without such ties.

def build_draft_tree(candidates, unary, edges, anchor, rows, chain_picks=None):
    """Returns dict(rows, copies, parent, depth, copy, token, path_length,
    path, expected, chain_expected) for one lane; candidates/unary [7][16],
    edges [7][16][16] (float32 arrays)."""
    import heapq
    import math
    C, P = 16, 7
    un = np.asarray(unary, np.float32).reshape(P, C)
    ed = np.asarray(edges, np.float32).reshape(P, C, C)
    cand = np.asarray(candidates, np.uint32).reshape(P, C)

    def score(p, k, j):
        return float(un[p, j]) + float(ed[p, k, j])

    def norm(p, k):
        top = max(score(p, k, j) for j in range(C))
        total = 0.0
        for j in range(C):
            total += math.exp(score(p, k, j) - top)
        return top + math.log(total)

    heap, seq = [], [0]

    def expand(parent, p, k, base, skip=None):
        n = norm(p, k)
        for j in range(C):
            if j != skip:
                heapq.heappush(heap, (-(base + score(p, k, j) - n), j, seq[0], p, parent))
                seq[0] += 1

    nodes = [dict(token=int(anchor), depth=0, pick=0, logp=0.0, chain=chain_picks is not None,
                  children=[])]
    if chain_picks is not None:
        parent, k, logp = 0, 0, 0.0
        for p in range(P):
            if len(nodes) >= rows:
                break
            pick = int(chain_picks[p])
            base = logp
            logp += score(p, k, pick) - norm(p, k)
            expand(parent, p, k, base, pick)
            nodes.append(dict(token=int(cand[p, pick]), depth=p + 1, pick=pick, logp=logp,
                              chain=True, children=[]))
            nodes[parent]["children"].append(len(nodes) - 1)
            parent, k = len(nodes) - 1, pick
    else:
        expand(0, 0, 0, 0.0)
    while len(nodes) < rows and heap:
        neg, pick, _, p, parent = heapq.heappop(heap)
        nodes.append(dict(token=int(cand[p, pick]), depth=p + 1, pick=pick, logp=-neg,
                          chain=False, children=[]))
        nodes[parent]["children"].append(len(nodes) - 1)
        if p + 1 < P:
            expand(len(nodes) - 1, p + 1, pick, -neg)
    out = dict(rows=len(nodes), copies=0, parent=[0] * 16, depth=[0] * 16, copy=[0] * 16,
               token=[0] * 16, path_length=[0] * 16, path=[[0] * 8 for _ in range(16)])
    assigned = [False] * 16
    stack, nxt = [], [0]

    def visit(node, parent_row):
        row = nxt[0]
        nxt[0] += 1
        out["parent"][row] = parent_row
        out["depth"][row] = nodes[node]["depth"]
        out["token"][row] = nodes[node]["token"]
        stack.append(row)
        kids = sorted(nodes[node]["children"],
                      key=lambda c: (not nodes[c]["chain"], -nodes[c]["logp"], nodes[c]["pick"]))
        if not kids:
            c = out["copies"]
            out["copies"] += 1
            out["path_length"][c] = len(stack)
            for i, r in enumerate(stack):
                out["path"][c][i] = r
            for r in stack:
                if not assigned[r]:
                    assigned[r] = True
                    out["copy"][r] = c
        for kid in kids:
            visit(kid, row)
        stack.pop()

    visit(0, 0)
    out["expected"] = sum(math.exp(n["logp"]) for n in nodes[1:])
    total, logp, k = 0.0, 0.0, 0
    for p in range(P):
        top, best = -math.inf, 0
        for j in range(C):
            s = score(p, k, j)
            if s > top:
                top, best = s, j
        ssum = 0.0
        for j in range(C):
            ssum += math.exp(score(p, k, j) - top)
        logp -= math.log(ssum)
        total += math.exp(logp)
        k = best
    out["chain_expected"] = total
    return out
