"""Benchmark of the MI355X logits->token step (one GPU).

Default: configuration C2 (the headline benchmark): one sampled step
over B=64 rows of V=151,936 fp32 logits with presence/frequency penalties over
2,048-token histories, T 0.7, top-k 50, top-p 0.9, one uniform per row. A
"step" is one jf_sample call over one batch; inputs are resident in HBM and
rotated over >= 512 MB of distinct copies so the 256 MB Infinity Cache cannot
serve a repeated step. Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 1..5]
"""
import argparse
import json
import os
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "justfit-llm_amd"))

PEAK_HBM_GBS = 8000.0
ROTATE_BYTES = 512 << 20


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--path", default="sample",
                    choices=["sample", "draft", "gather", "verify"],
                    help="sample: jf_sample on --config (the headline); draft: "
                         "jf_draft_select at 4 lanes, V=151936; gather: jf_tree_gather "
                         "of one KV-like tensor family after C4's tree acceptance; verify: "
                         "the engine's penalized chain verify (4 lanes x 16 rows, "
                         "V=248320, extras and sparse drafts) plus chain acceptance")
    ap.add_argument("--mode", default="auto",
                    help="C3/C4: greedy or sampled (auto: sampled); C2: general runs "
                         "C2's batch through the general kernels (rows one float past "
                         "16-byte alignment, top-k 3000: select_kernel, merge_kernel "
                         "and the multi-pass stages)")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="bound of the CPU-baseline sample")
    ap.add_argument("--history", default="uniform", choices=["uniform", "zipf", "mixed"],
                    help="C2 only: zipf gives every row a history clustered in low ids "
                         "(Zipf 1.2, about 450 distinct ids in the first chunk, past 256 "
                         "fixed penalty slots: the table widens to 512 a chunk); mixed "
                         "does so for every fourth row")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 64 MiB device copy (20 times): the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE readings to bytes")
    return ap.parse_args()


def build_workload(cfg, mode, history="uniform"):
    """Host inputs, per-row policies and the algorithmic bytes of one step."""
    import jf_sampler as J
    from jf_sampler import workloads as WL
    w = {}
    if cfg == 1:
        c = WL.config1()
        w.update(V=c["V"], logits=c["logits"], policies=[J.policy(**c["policy"])],
                 histories=c["histories"], generated=c["generated"], mark_prompt=True,
                 name="C1 greedy B=1 V=151936 fp32 repetition 1.1 over 256 prompt ids",
                 dtype="f32")
        hist_bytes = 256 * 4
    elif cfg == 2:
        c = WL.config2()
        B = c["logits"].shape[0]
        hists, label = c["histories"], "2048 ids"
        if history != "uniform":
            # Ids clustered near 0 as real text's are: about 450 distinct ids
            # below 8192, past the first chunk's 256 fixed slots (the table
            # widens to 512).
            rng = np.random.default_rng(22)
            every = 1 if history == "zipf" else 4
            hists = [np.minimum(rng.zipf(1.2, len(h)) - 1, c["V"] - 1).astype(np.uint32)
                     if r % every == 0 else h for r, h in enumerate(hists)]
            label = ("2048 Zipf(1.2)-clustered ids" if every == 1 else
                     "2048 ids, every 4th row Zipf(1.2)-clustered")
        pol = dict(c["policy"])
        name = ("C2 sampled B=64 V=151936 fp32 T0.7 top-k 50 top-p 0.9 "
                f"presence 0.5 frequency 0.3 over {label}")
        if mode == "general":
            # The kernels a call takes when the fast pass and the small merge
            # cannot: rows whose logits start one float past a 16-byte
            # boundary (an engine's views into a padded buffer) and a top-k
            # past the merge's lists.
            pol["top_k"] = 3000
            w["unaligned"] = True
            w["kernel"] = "jf::select_kernel<0>"
            name = name.replace("top-k 50", "top-k 3000") + ", rows 4 bytes past alignment"
        w.update(V=c["V"], logits=c["logits"], policies=[J.policy(**pol)] * B,
                 histories=hists, generated=c["generated"], mark_prompt=False,
                 uniforms=c["uniforms"], name=name, dtype="f32")
        hist_bytes = B * 2048 * 4
    elif cfg == 3:
        c = WL.config3()
        B = c["logits_bf16"].shape[0]
        sampled = mode != "greedy"
        p = J.policy(temperature=1.0, constrained=True) if sampled else J.policy(constrained=True)
        w.update(V=c["V"], logits_bf16=c["logits_bf16"], masks=c["masks"], policies=[p] * B,
                 uniforms=c["uniforms"],
                 name=f"C3 grammar B=32 V=151936 bf16 mask u32[32][4748] "
                      f"{'T1.0 sampled' if sampled else 'greedy'}",
                 dtype="bf16->f32")
        hist_bytes = c["masks"].nbytes
        if sampled:
            # Every row keeps every admitted token: the select launch draws it.
            w["kernel"] = "jf::select_fast_kernel<1, false, jf::NoRows, jf::UncutFinish>"
    elif cfg == 4:
        c = WL.config4()
        rows = c["logits"].shape[0]
        sampled = mode != "greedy"
        pol = J.policy(temperature=1.0) if sampled else J.policy()
        w.update(V=c["V"], logits=c["logits"], policies=[pol] * rows,
                 name=f"C4 tree verify 16x16 nodes V=151936 fp32 "
                      f"{'rejection sampling (dense q)' if sampled else 'greedy'}"
                      " + tree acceptance",
                 dtype="f32", tree=c, sampled=sampled)
        hist_bytes = c["q"].nbytes if sampled else 0
        if sampled:
            w["uniforms"] = c["uniforms"]
            # The select pass also stores the drafted rows' weights for
            # their residual pass.
            w["kernel"] = "jf::select_fast_kernel<0, false, jf::NoRows, jf::StoreWeights>"
    else:
        c = WL.config5()
        B = c["logits_bf16"].shape[0]
        w.update(V=c["V"], logits_bf16=c["logits_bf16"], policies=[J.policy(**c["policy"])] * B,
                 histories=c["histories"], generated=c["generated"], mark_prompt=True,
                 uniforms=c["uniforms"],
                 name="C5 large B=256 V=248320 bf16 min-p 0.05 top-k 1000 top-p 0.95 "
                      "T0.8 penalties over 8192 ids",
                 dtype="bf16->f32")
        hist_bytes = B * 8192 * 4
    lg = w.get("logits", w.get("logits_bf16"))
    rows = lg.shape[0]
    w["rows"] = rows
    w["alg_bytes"] = lg.nbytes + hist_bytes + rows * 4 * 2  # + uniforms + outputs
    # The select kernel reads the logits and the history ids or mask words;
    # C4's dense draft q is read only by the residual pass (C4 sampled's
    # select also writes the drafted rows' weights for that pass: traffic
    # beyond these bytes).
    w["select_bytes"] = lg.nbytes + (0 if cfg == 4 else hist_bytes)
    return w


class GpuStep:
    """Device-resident inputs (rotated copies) and one jf_sample per step."""

    def __init__(self, w, count_headroom=0):
        import torch
        import jf_sampler as J
        self.w = w
        dev = torch.device("cuda", 0)
        V, rows = w["V"], w["rows"]
        host = w.get("logits")
        if host is not None:
            base = torch.from_numpy(host)
        else:
            base = torch.from_numpy(w["logits_bf16"].view(np.int16)).view(torch.bfloat16)
        per = base.numel() * base.element_size()
        copies = max(2, -(-ROTATE_BYTES // per))
        if w.get("unaligned"):
            # Each row one element past its buffer row's start.
            def shifted():
                t = torch.empty((base.shape[0], base.shape[1] + 1), dtype=base.dtype, device=dev)
                t[:, 1:] = base.to(dev)
                return t[:, 1:]
            self.copies = [shifted() for _ in range(copies)]
        else:
            self.copies = [base.to(dev) for _ in range(copies)]
        self.sampler = J.Sampler(V, rows)
        self.kw = []
        self.tables = []
        extra = {}
        if "masks" in w:
            extra["masks"] = torch.from_numpy(w["masks"].view(np.int32)).to(dev)
        if "uniforms" in w:
            u = w["uniforms"]
            if u.ndim == 2:  # C4: per-row uniform slot 24 + r of each request
                rq = u.shape[0]
                idx = np.array([k * 40 + 24 + r for k in range(rq) for r in range(rows // rq)],
                               np.uint32)
                extra["uniform_index"] = torch.from_numpy(idx.view(np.int32)).to(dev)
                u = u.reshape(-1)
            extra["uniforms"] = torch.from_numpy(np.ascontiguousarray(u)).to(dev)
        if w.get("tree") is not None and w.get("sampled"):
            c = w["tree"]
            from jf_sampler import workloads as WL
            draft = np.full(rows, 0xFFFFFFFF, np.uint32)
            for k, parent in enumerate(c["trees"]):
                n = WL.chain_length(parent)
                for r in range(n - 1):
                    draft[k * 16 + r] = c["tokens"][k][r + 1]
            extra["draft_tokens"] = torch.from_numpy(draft.view(np.int32)).to(dev)
            # The engine builds its trees on the host (jf_build_draft_tree),
            # so it names the drafted rows, each lane's chain
            # (Runtime.cpp:1284-1306 passes chain_rows per lane), as the
            # row-indexed call does; the other rows draw plainly.
            extra["draft_token_index"] = [r if draft[r] != 0xFFFFFFFF else 0xFFFFFFFF
                                          for r in range(rows)]
            self.q = [torch.from_numpy(c["q"]).to(dev) for _ in range(len(self.copies))]
            extra["out_draft_probs"] = torch.zeros(rows, dtype=torch.float32, device=dev)
        self.draft_probs = extra.get("out_draft_probs")
        self.extra = extra  # the device tensors the argument records point at
        self.out = torch.zeros(rows, dtype=torch.int32, device=dev)
        # C4's step ends as the engine's does: tree acceptance over the
        # selected tokens (tree.metal:20-84; Runtime.cpp:1284-1306), which
        # rewrites them in place into each request's accepted path.
        self.accept = None
        if w.get("tree") is not None:
            c = w["tree"]
            from jf_sampler import workloads as WL
            rq, per = len(c["trees"]), rows // len(c["trees"])
            sampled = w.get("sampled")
            trees = []
            for k in range(rq):
                if sampled:
                    n = WL.chain_length(c["trees"][k])
                    cq = [float(c["q"][k * per + j, c["tokens"][k][j + 1]]) for j in range(n - 1)]
                    trees.append(J.tree_lane(c["trees"][k], c["tokens"][k], n, cq))
                else:
                    trees.append(J.tree_lane(c["trees"][k], c["tokens"][k]))
            self.acc_out = [torch.zeros(rq, dtype=torch.int32, device=dev) for _ in range(2)]
            self.acc_path = torch.zeros((rq, 8), dtype=torch.int32, device=dev)
            kw_acc = dict(trees=trees, rows_per_lane=per, target_tokens=self.out.view(rq, per),
                          retained=self.acc_out[0], accepted=self.acc_out[1],
                          path_rows=self.acc_path, maximum_retained=[8] * rq,
                          policies=[w["policies"][0]] * rq)
            if sampled:
                self.acc_u = torch.from_numpy(np.ascontiguousarray(c["uniforms"])).to(dev)
                kw_acc.update(target_draft_probs=self.draft_probs.view(rq, per),
                              uniforms=self.acc_u)
            self.acc_trees = trees
            self.accept = ("tree",) + self.sampler.accept_tree_args(**kw_acc)
        for i in range(len(self.copies)):
            kw = dict(extra)
            if "histories" in w:
                H = max(len(h) for h in w["histories"])
                t = J.PenaltyTable(V, rows, H + 8 + count_headroom)
                for r, h in enumerate(w["histories"]):
                    t.rebuild(r, h, w["generated"][r], None, w["mark_prompt"])
                self.tables.append(t)
                kw["penalties"] = t
                kw["penalty_rows"] = list(range(rows))
            if w.get("tree") is not None and w.get("sampled"):
                kw["dense_q"] = self.q[i]
            a, keep = self.sampler.sample_args(self.copies[i], w["policies"], self.out, **kw)
            self.kw.append((a, keep))
        torch.cuda.synchronize()

    def step(self, i):
        a, _ = self.kw[i % len(self.kw)]
        if self.accept is not None and self.accept[0] == "tree":
            # Selection and tree acceptance in one call (one launch when the
            # lanes are greedy).
            self.sampler.launch_sample_accept_tree(a, self.accept[1])
            return
        self.sampler.launch(a)
        if self.accept is not None:
            self.sampler.launch_accept(self.accept)


class VerifyStep:
    """The engine's penalized chain-verify step (Sampling::addVerify then
    addAcceptance, Sampling.cpp:149-172, 278-328): one jf_sample over every
    lane's 16 verify rows, addressed per row (draft token, candidate row,
    extra penalty tokens), then jf_accept_chain over the lanes, which
    rewrites the selected tokens into each lane's accepted chain. Inputs
    resident and rotated like GpuStep's."""

    def __init__(self, c):
        import torch
        import jf_sampler as J
        dev = torch.device("cuda", 0)
        V, lanes, rows = c["V"], c["lanes"], c["rows"]
        B = lanes * rows
        pol = J.policy(**c["policy"])
        self.c = c
        self.w = dict(V=V, rows=B, policies=[pol] * B, dtype="f32",
                      name=f"verify {lanes} lanes x {rows} rows V={V} fp32, T0.7 top-k 50 "
                           "top-p 0.9 repetition 1.1 presence 0.5 frequency 0.3 over 2048 ids "
                           "+ verify extras, 16 sparse candidates a proposal, then chain "
                           "acceptance")
        base = torch.from_numpy(c["logits"])
        per = base.numel() * base.element_size()
        self.copies = [base.to(dev) for _ in range(max(2, -(-ROTATE_BYTES // per)))]
        self.sampler = J.Sampler(V, B)
        t32 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int32)).to(dev)
        self.inputs = t32(c["inputs"])
        self.cand = t32(c["cand_ids"])
        self.cprob = torch.from_numpy(c["cand_probs"]).to(dev)
        self.u = torch.from_numpy(np.ascontiguousarray(c["uniforms"].reshape(-1))).to(dev)
        self.uidx = t32(c["uniform_index"])
        self.proposed = t32(c["inputs"].reshape(lanes, rows)[:, 1:])
        self.out = torch.zeros(B, dtype=torch.int32, device=dev)
        self.draft_probs = torch.zeros(B, dtype=torch.float32, device=dev)
        self.retained = torch.zeros(lanes, dtype=torch.int32, device=dev)
        self.accepted = torch.zeros(lanes, dtype=torch.int32, device=dev)
        H = max(len(h) for h in c["histories"])
        self.tables, self.kw = [], []
        for x in self.copies:
            t = J.PenaltyTable(V, lanes, H + 8)
            for l, h in enumerate(c["histories"]):
                t.rebuild(l, h, c["generated"][l], None, c["mark_prompt"])
            self.tables.append(t)
            self.kw.append(self.sampler.sample_args(
                x, self.w["policies"], self.out, penalties=t,
                penalty_rows=[g // rows for g in range(B)], extra_tokens=self.inputs,
                extra_counts=list(c["extra_counts"]), uniforms=self.u,
                uniform_index=self.uidx, draft_tokens=self.inputs, cand_ids=self.cand,
                cand_probs=self.cprob, out_draft_probs=self.draft_probs,
                draft_token_index=c["draft_index"], draft_cand_index=c["cand_index"],
                extra_offsets=c["extra_offsets"]))
        self.accept = ("chain",) + self.sampler.accept_chain_args(
            verify_rows=rows, proposed=self.proposed, target_tokens=self.out,
            retained=self.retained, accepted=self.accepted, maximum_retained=[rows] * lanes,
            policies=[pol] * lanes, candidates=self.cand, proposal_probs=self.cprob,
            target_draft_probs=self.draft_probs, uniforms=self.u)
        torch.cuda.synchronize()

    def step(self, i):
        a, _ = self.kw[i % len(self.kw)]
        self.sampler.launch(a)
        self.sampler.launch_accept(self.accept)

    def close(self):
        for t in self.tables:
            t.close()
        self.sampler.close()


class HipEvents:
    """Raw HIP events (libamdhip64 through ctypes) for the library to record
    around its selection kernel."""

    def __init__(self, n):
        import ctypes
        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            rc = self.hip.hipEventCreate(ctypes.byref(e))
            assert rc == 0, f"hipEventCreate: {rc}"
            self.ev.append(e)

    def ms(self, i, j):
        out = self.ct.c_float()
        rc = self.hip.hipEventElapsedTime(self.ct.byref(out), self.ev[i], self.ev[j])
        assert rc == 0, f"hipEventElapsedTime: {rc}"
        return out.value

    def destroy(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


def time_select(g, first, steps):
    """The selection kernel's own duration: a pair of HIP events that the
    library's launch of that kernel records at its start and end
    (hipExtLaunchKernelGGL) on the stream it runs on. Returns the mean and
    p50 in microseconds."""
    import torch
    ev = HipEvents(2 * steps)
    torch.cuda.synchronize()
    for i in range(steps):
        a, _ = g.kw[(first + i) % len(g.kw)]
        a.select_start_event = ev.ev[2 * i].value
        a.select_done_event = ev.ev[2 * i + 1].value
        g.sampler.launch(a)
        a.select_start_event = None
        a.select_done_event = None
    torch.cuda.synchronize()
    us = np.array([ev.ms(2 * i, 2 * i + 1) for i in range(steps)]) * 1000.0
    ev.destroy()
    return float(us.mean()), float(np.percentile(us, 50))


def time_with_counts(g, steps):
    """Steps each followed by the engine's commit of one token per row into
    the penalty table (jf_penalty_table_count_rows: an in-place device update
    on the same stream, no upload). The tokens are a fixed synthetic
    sequence; each step's table is the one its input copy reads."""
    import torch
    rows = g.w["rows"]
    rng = np.random.default_rng(99)
    idx = np.arange(rows, dtype=np.uint32)
    toks = rng.integers(0, g.w["V"], (steps, rows), dtype=np.uint32)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(steps):
        g.step(i)
        g.tables[i % len(g.tables)].count_rows(idx, toks[i])
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]) * 1000.0
    return {"ms_per_step": ev[0].elapsed_time(ev[steps]) / steps,
            "p50_us": float(np.percentile(per, 50)),
            "note": "each step followed by jf_penalty_table_count_rows of one token per row"}


def accept_ptr(g, kind):
    """The step's prepared acceptance record of `kind` ("chain" or "tree"),
    as a pointer for the C++ loop, or None."""
    import ctypes
    acc = getattr(g, "accept", None)
    if acc is None or acc[0] != kind:
        return None
    return ctypes.cast(ctypes.pointer(acc[1]), ctypes.c_void_p)


def time_cpp_loop(g, steps, with_counts, batch=0):
    """The same calls issued from C++ (libjf_bench_loop.so), as a native
    engine issues them: GPU and host microseconds per step without the
    Python loop, optionally with the per-step penalty count, and with
    `batch` the mean step time of each run of that many steps."""
    import ctypes
    import jf_sampler as J
    J.lib()  # the sampler library first: one HIP runtime in the process
    L = ctypes.CDLL(os.path.join(REPO, "justfit-llm_amd", "jf_sampler", "libjf_bench_loop.so"))
    vp, u32 = ctypes.c_void_p, ctypes.c_uint32
    L.jf_bench_sample_loop.argtypes = [vp, vp, u32, u32, vp, vp, vp, u32, vp,
                                       ctypes.POINTER(ctypes.c_double),
                                       ctypes.POINTER(ctypes.c_double), u32, vp, vp, vp,
                                       ctypes.c_int]
    n = len(g.kw)
    arr = (J.JfSampleArgs * n)(*[a for a, _ in g.kw])
    rows = g.w["rows"]
    tables = idx = toks = None
    if with_counts:
        tables = (vp * n)(*[t.handle.value for t in g.tables])
        idx = np.arange(rows, dtype=np.uint32)
        toks = np.random.default_rng(98).integers(0, g.w["V"], (steps, rows), dtype=np.uint32)
    batch_us = np.zeros(steps // batch, np.float32) if batch else None
    gpu, host = ctypes.c_double(), ctypes.c_double()
    rc = L.jf_bench_sample_loop(g.sampler.handle, ctypes.cast(arr, vp), n, steps, tables,
                                None if idx is None else idx.ctypes.data_as(vp),
                                None if toks is None else toks.ctypes.data_as(vp), rows,
                                J._stream(), ctypes.byref(gpu), ctypes.byref(host), batch,
                                None if batch_us is None else batch_us.ctypes.data_as(vp),
                                accept_ptr(g, "chain"), accept_ptr(g, "tree"), 1)
    if rc:
        raise RuntimeError(f"C++ timing loop failed: {rc} {J.lib().jf_last_error().decode()}")
    out = {"us_per_step": gpu.value, "host_us_per_call": host.value}
    if batch:
        out["batch_us"] = batch_us
    return out


def host_issue_us(g, bursts=20, per=16):
    """The host's own cost of issuing one step: bursts of `per` steps from
    C++, each started on an idle stream, timed on the host only. A burst
    stays far below the depth of the device queue, so no call waits for the
    GPU (in a long loop the host runs ahead until the queue is full and then
    issues at the GPU's pace, which the long loop's host time shows).
    Returns the median over the bursts, in microseconds per step."""
    import torch
    vals = []
    for _ in range(bursts):
        torch.cuda.synchronize()
        vals.append(time_cpp_loop(g, per, False)["host_us_per_call"])
    torch.cuda.synchronize()
    return float(np.median(vals))


def pick_batch(steps):
    """Steps per timed run for the step-time distribution: the largest
    divisor of `steps` up to 25 that leaves at least four runs, else at least
    two (1 when none does)."""
    for runs in (4, 2):
        for d in range(min(25, steps // runs), 1, -1):
            if steps % d == 0:
                return d
    return 1


def time_cpp_calls(kind, argv, steps, batch=0, selector=None):
    """jf_draft_select on `selector` (kind "draft") or jf_tree_gather (kind
    "gather") over the prepared argument records `argv` (rotated), issued
    back to back from C++ (libjf_bench_loop.so): GPU and host microseconds
    per step, and with `batch` the mean step time of each run of that many
    steps."""
    import ctypes
    import jf_sampler as J
    J.lib()  # the sampler library first: one HIP runtime in the process
    L = ctypes.CDLL(os.path.join(REPO, "justfit-llm_amd", "jf_sampler", "libjf_bench_loop.so"))
    vp, u32, dp = ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_double)
    n = len(argv)
    arr = (type(argv[0]) * n)(*argv)
    batch_us = np.zeros(steps // batch, np.float32) if batch else None
    gpu, host = ctypes.c_double(), ctypes.c_double()
    tail = (J._stream(), ctypes.byref(gpu), ctypes.byref(host), batch,
            None if batch_us is None else batch_us.ctypes.data_as(vp))
    if kind == "draft":
        f = L.jf_bench_draft_loop
        f.argtypes = [vp, vp, u32, u32, vp, dp, dp, u32, vp]
        rc = f(selector.handle, ctypes.cast(arr, vp), n, steps, *tail)
    else:
        f = L.jf_bench_gather_loop
        f.argtypes = [vp, u32, u32, vp, dp, dp, u32, vp]
        rc = f(ctypes.cast(arr, vp), n, steps, *tail)
    if rc:
        raise RuntimeError(f"C++ timing loop failed: {rc} {J.lib().jf_last_error().decode()}")
    out = {"us_per_step": gpu.value, "host_us_per_call": host.value}
    if batch:
        out["batch_us"] = batch_us.astype(np.float64)
    return out


def time_python_calls(call, argv, steps):
    """The same calls from a Python/ctypes loop, between events at the
    loop's ends: microseconds per step."""
    import torch
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for i in range(steps):
        call(argv[i % len(argv)])
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1000.0 / steps


def time_graph(g, steps):
    """Steps captured in a HIP graph and replayed: jf_sample_static (the
    entry point that allocates nothing; row parameters travel as kernel
    arguments) over pick_batch(steps) rotated input copies per graph, the
    graph replayed until `steps` steps have run, between HIP events. None
    where the static entry point's limits (64 rows, 262,144 tokens) exclude
    the workload."""
    import torch
    import jf_sampler as J
    V, rows = g.w["V"], g.w["rows"]
    if rows > 64 or V > 262144:
        return None
    per = pick_batch(steps)
    args = [g.kw[i % len(g.kw)][0] for i in range(per)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        J.sample_static(V, args[0])  # the scratch address lookup, outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for a in args:
            J.sample_static(V, a)
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps // per):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / steps
    del graph
    return {"us_per_step": us,
            "note": f"jf_sample_static captured {per} steps to a HIP graph, replayed "
                    f"{steps // per} times"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, seconds):
    """The oracle (a C restatement, pthreads over rows) built here with -O3
    -march=native, timed step by step: 3 warm-up steps, then the median of
    up to 20 timed steps (fewer when 20 would pass `seconds`). Its tokens
    must equal the -O2 checker build's on the same step."""
    import tempfile
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    if w.get("tree") is not None and w.get("sampled"):
        return None  # the dense-residual draw is not in the batch driver
    V, rows = w["V"], w["rows"]
    # The pool's CPU share for one GPU is 16 cores, whatever the affinity shows.
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    native_dir = tempfile.mkdtemp(prefix="jf_oracle_native_")
    L = O.native_lib(native_dir)
    pols = [O.policy_from(p) for p in w["policies"]]
    words, pen_rows = None, None
    if "histories" in w:
        words = np.zeros((rows, V), np.uint32)
        for r, h in enumerate(w["histories"]):
            rc, words[r] = O.rebuild_penalty_words(V, h, w["generated"][r], None, w["mark_prompt"])
        pen_rows = np.arange(rows, dtype=np.uint32)
    is_bf16 = "logits_bf16" in w
    lg = w["logits_bf16"] if is_bf16 else w["logits"]
    u = w.get("uniforms")
    if u is not None and u.ndim == 2:
        u = None

    def step(library):
        return O.select_batch(V, pols, lg, is_bf16=is_bf16, masks=w.get("masks"),
                              words=words, pen_rows=pen_rows, uniforms=u,
                              threads=threads, library=library)[0]

    want = step(None)
    for _ in range(3):
        got = step(L)
    if not np.array_equal(got, want):
        raise RuntimeError("the -O3 -march=native oracle build disagrees with the checker build")
    times = []
    t0 = time.perf_counter()
    while len(times) < 20:
        t = time.perf_counter()
        step(L)
        times.append(time.perf_counter() - t)
        if time.perf_counter() - t0 >= seconds and len(times) >= 5:
            break
    med = float(np.median(times))
    model = cpu_model()
    return dict(value=1.0 / med, unit="steps/s", cores=threads, kind="port",
                cpu_model=model,
                sample=f"median of {len(times)} timed full steps ({rows} rows each, after "
                       f"3 warm-ups) of the same seeded workload: {med * 1e3:.1f} ms/step; "
                       f"oracle/jf_oracle.c built with -O3 -march=native "
                       f"-ffp-contract=off on this host ({model}), {threads} threads "
                       f"over rows; tokens equal to the -O2 checker build's")


# The committed rocprofv3 summary of each workload (profiles/<name>.txt): one
# line per kernel with its trace statistics and HBM traffic.
PROFILE_NAMES = {(1, "auto"): "select_c1", (2, "auto"): "select_merge_c2",
                 (3, "greedy"): "select_c3_greedy", (3, "sampled"): "select_uncut_c3_sampled",
                 (4, "greedy"): "select_c4_greedy", (4, "sampled"): "select_uncut_c4_sampled",
                 (5, "auto"): "select_merge_c5", (2, "zipf"): "select_merge_c2_zipf",
                 (2, "mixed"): "select_merge_c2_mixed", ("draft", "auto"): "draft_select",
                 ("gather", "auto"): "tree_gather", ("verify", "auto"): "select_verify",
                 (2, "general"): "select_general_c2"}


def profile_key(cfg, mode, history="uniform"):
    if cfg in (3, 4):
        return (cfg, "greedy" if mode == "greedy" else "sampled")
    if cfg == 2 and history != "uniform":
        return (cfg, history)
    if cfg == 2 and mode == "general":
        return (cfg, "general")
    return (cfg, "auto")


def profile_row(key, kernel):
    """The fields of `kernel`'s line in the workload's summary, or None."""
    name = PROFILE_NAMES.get(key)
    path = os.path.join(REPO, "profiles", f"{name}.txt") if name else None
    if not kernel or not path or not os.path.exists(path):
        return None
    for line in open(path):
        # The name may hold spaces (template arguments); the fields follow it.
        if line.startswith(kernel + " "):
            return [kernel] + line[len(kernel):].split()
    return None


def read_traffic(key, kernel):
    """HBM bytes per launch of `kernel` (FETCH_SIZE and WRITE_SIZE scaled by a
    copy kernel's readings) from the committed summary, or None."""
    f = profile_row(key, kernel)
    try:
        return float(f[7]) if f and f[7] != "-" else None
    except (IndexError, ValueError):
        return None


def read_profile_us(key, kernel):
    """The kernel's rocprofv3 average duration (us) in the committed summary
    of the same workload, or None."""
    f = profile_row(key, kernel)
    try:
        return float(f[2]) if f else None
    except (IndexError, ValueError):
        return None


def copy_calibration():
    import torch
    n = 64 << 20
    src = torch.ones(n // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n, "bytes_written": n, "launches": 20}))


def bench_draft(args):
    """The draft selector (jf_draft_select) at the reference's widest batch:
    4 lanes x 7 proposal positions over V=151936 fp32 draft logits, inputs
    resident and rotated over >= 512 MB. The dominant kernel is the top-16
    pass over the proposal rows (draft_top16_kernel)."""
    import torch
    import jf_sampler as J
    from jf_sampler import workloads as WL
    c = WL.config_draft()
    lanes, V = c["lanes"], c["V"]
    print(f"# draft selector {lanes} lanes V={V}: building inputs", file=sys.stderr, flush=True)
    dev = torch.device("cuda", 0)
    base = torch.from_numpy(c["logits"])
    copies = [base.to(dev) for _ in range(max(2, -(-ROTATE_BYTES // (base.numel() * 4))))]
    t16 = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)
    hidden, pred, succ = t16(c["hidden"]), t16(c["pred"]), t16(c["succ"])
    u = torch.from_numpy(c["uniforms"]).to(dev)
    cand = torch.zeros((lanes * 7, 16), dtype=torch.int32, device=dev)
    unary = torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev)
    tokens = torch.zeros(lanes * 7, dtype=torch.int32, device=dev)
    q = torch.zeros((lanes * 7, 16), dtype=torch.float32, device=dev)
    sel = J.DraftSelector(V, lanes)
    pols = [J.policy(temperature=t) for t in c["temperatures"]]
    argv = [sel.args(logits=x, hidden=hidden, pred_codebook=pred, succ_codebook=succ,
                     anchors=c["anchors"], policies=pols, candidates=cand, unary=unary,
                     tokens=tokens, q=q, uniforms=u) for x in copies]
    for i in range(args.warmup):
        sel.launch(argv[i % len(argv)])
    torch.cuda.synchronize()
    K = args.steps
    wall0 = time.perf_counter()
    cpp = time_cpp_calls("draft", argv, K, selector=sel)
    wall = time.perf_counter() - wall0
    ms_per_step = cpp["us_per_step"] / 1000.0
    per = time_cpp_calls("draft", argv, K, batch=pick_batch(K), selector=sel)["batch_us"]
    py_us = time_python_calls(sel.launch, argv, K)
    # The top-16 kernel alone, between events its launch records.
    hev = HipEvents(2 * K)
    for i in range(K):
        a = argv[(args.warmup + i) % len(argv)]
        a.select_start_event, a.select_done_event = hev.ev[2 * i].value, hev.ev[2 * i + 1].value
        sel.launch(a)
        a.select_start_event = a.select_done_event = None
    torch.cuda.synchronize()
    kus = np.array([hev.ms(2 * i, 2 * i + 1) for i in range(K)]) * 1000.0
    hev.destroy()
    top_bytes = lanes * 7 * V * 4
    achieved = top_bytes / (kus.mean() * 1e-6) / 1e9
    kernel = "jf::draft_top16_kernel<true>"
    traffic = read_traffic(("draft", "auto"), kernel)
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O
        sampled = [t > 0 for t in c["temperatures"]]
        steps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            O.draft_select(c["logits"], c["hidden"], c["pred"], c["succ"], c["anchors"],
                           c["temperatures"], sampled, c["uniforms"])
            steps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=steps / el, unit="selections/s", cores=1, kind="port",
                   sample=f"{steps} full selections ({lanes} lanes x 7 positions) of the same "
                          f"seeded inputs in {el:.1f} s, oracle/jf_oracle.c -O2, one thread")
    line = {
        "metric": "draft selections/sec at 4 lanes x 7 positions, V=151936; achieved HBM GB/s "
                  "vs peak; p50 us/selection",
        "value": 1000.0 / ms_per_step, "unit": "selections/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": ms_per_step,
        "p50_us": float(np.percentile(per, 50)), "p90_us": float(np.percentile(per, 90)),
        "wall_s": wall, "host_us_per_call": cpp["host_us_per_call"], "python_loop_us": py_us,
        "timing": "jf_draft_select called back to back from C++ (libjf_bench_loop.so), HIP "
                  "events at the loop's ends; p50/p90 over runs of pick_batch(K) steps",
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": f"synthetic (workloads.config_draft), {len(copies)} rotated "
                                f"logits copies >= 512 MB",
        "config": {"workload": f"draft selector {lanes} lanes x 7 positions V={V} fp32, "
                               "bf16 codebooks rank 256, lanes alternate greedy / T0.8",
                   "rows": lanes * 7, "vocabulary": V, "algorithmic_bytes_per_step": top_bytes},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "kernel": kernel,
                     "kernel_mean_us": float(kus.mean()),
                     "kernel_p50_us": float(np.percentile(kus, 50)),
                     "algorithmic_bytes": top_bytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    sel.close()


def bench_gather(args):
    """The tree gather (jf_tree_gather) of one KV-like tensor family: 16
    lanes (C4's requests) x 16 verify rows, 36 layers x 1024 bf16 columns
    per row (8 KV heads x 128), each lane's accepted path (ascending, depth
    <= 8) moved to its first rows. Algorithmic bytes: each moved element read
    and written once."""
    import torch
    import jf_sampler as J
    sys.path.insert(0, os.path.join(REPO, "tests"))
    from gather_cases import gather_case
    rng = np.random.default_rng(7)
    data, path, retained, p = gather_case(rng, lanes=16, layers=36, rows=16, columns=1024,
                                          inner=1024, pad=0)
    moved = sum(1 for b in range(p["lanes"]) for i in range(min(int(retained[b]), 8))
                if int(path[b, i]) != i)
    alg = moved * p["layers"] * p["columns"] * 2 * 2
    print(f"# tree gather {p}: {moved} moved rows", file=sys.stderr, flush=True)
    dev = torch.device("cuda", 0)
    base = torch.from_numpy(data.view(np.int16))
    copies = [base.to(dev) for _ in range(max(2, -(-ROTATE_BYTES // data.nbytes)))]
    pr = torch.from_numpy(path.view(np.int32)).to(dev)
    rt = torch.from_numpy(retained.view(np.int32)).to(dev)
    argv = [J.tree_gather_args(c, pr, rt, **p) for c in copies]
    for i in range(args.warmup):
        J.tree_gather(argv[i % len(argv)])
    torch.cuda.synchronize()
    K = args.steps
    wall0 = time.perf_counter()
    cpp = time_cpp_calls("gather", argv, K)
    wall = time.perf_counter() - wall0
    ms_per_step = cpp["us_per_step"] / 1000.0
    per = time_cpp_calls("gather", argv, K, batch=pick_batch(K))["batch_us"]
    py_us = time_python_calls(J.tree_gather, argv, K)
    hev = HipEvents(2 * K)
    for i in range(K):
        a = argv[(args.warmup + i) % len(argv)]
        a.start_event, a.done_event = hev.ev[2 * i].value, hev.ev[2 * i + 1].value
        J.tree_gather(a)
        a.start_event = a.done_event = None
    torch.cuda.synchronize()
    kus = np.array([hev.ms(2 * i, 2 * i + 1) for i in range(K)]) * 1000.0
    hev.destroy()
    achieved = alg / (kus.mean() * 1e-6) / 1e9
    kernel = "jf::tree_gather_kernel<true>"
    traffic = read_traffic(("gather", "auto"), kernel)
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(REPO, "oracle"))
        import oracle as O
        steps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            O.tree_gather(data, path, retained, **p)
            steps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=steps / el, unit="gathers/s", cores=1, kind="port",
                   sample=f"{steps} whole gathers of the same inputs in {el:.1f} s (each "
                          f"includes a {data.nbytes >> 20} MiB copy of the tensor), "
                          f"oracle/jf_oracle.c -O2, one thread")
    line = {
        "metric": "tree gathers/sec of one KV-like family (16 lanes x 16 rows, 36 layers x "
                  "1024 bf16); achieved HBM GB/s vs peak; p50 us/gather",
        "value": 1000.0 / ms_per_step, "unit": "gathers/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": ms_per_step,
        "p50_us": float(np.percentile(per, 50)), "p90_us": float(np.percentile(per, 90)),
        "wall_s": wall, "host_us_per_call": cpp["host_us_per_call"], "python_loop_us": py_us,
        "timing": "jf_tree_gather called back to back from C++ (libjf_bench_loop.so), HIP "
                  "events at the loop's ends; p50/p90 over runs of pick_batch(K) steps",
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u16", "data": f"synthetic (tests/gather_cases.py, seed 7), {len(copies)} rotated "
                                f"copies >= 512 MB",
        "config": {"workload": "tree gather 16 lanes x 16 rows x 36 layers x 1024 columns bf16",
                   "moved_rows": moved, "algorithmic_bytes_per_step": alg},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic,
                     "kernel": kernel,
                     "kernel_mean_us": float(kus.mean()),
                     "kernel_p50_us": float(np.percentile(kus, 50)), "algorithmic_bytes": alg},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def verify_cpu_baseline(c, seconds):
    """The oracle (C restatement, one thread) over whole verify steps: every
    row's selection (jfo_select_row with its extras, draft and candidates)
    and each lane's chain acceptance, repeated for about `seconds`."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    V, lanes, rows = c["V"], c["lanes"], c["rows"]
    pol = O.policy(**c["policy"])
    words = [O.rebuild_penalty_words(V, h, c["generated"][l], None, c["mark_prompt"])[1]
             for l, h in enumerate(c["histories"])]
    inp = c["inputs"]

    def step():
        vt = np.zeros(lanes * rows, np.uint32)
        vp = np.zeros(lanes * rows, np.float32)
        for l in range(lanes):
            for r in range(rows):
                g = l * rows + r
                d = int(c["draft_index"][g])
                ci = int(c["cand_index"][g])
                vt[g], vp[g] = O.select_row(
                    V, pol, logits=c["logits"][g], words=words[l],
                    extra=inp[l * rows + 1:l * rows + 1 + r],
                    uniform=float(c["uniforms"][l, 15]),
                    draft_token=int(inp[d]) if d != 0xFFFFFFFF else O.NO_TOKEN,
                    cand_ids=c["cand_ids"][ci] if d != 0xFFFFFFFF else None,
                    cand_probs=c["cand_probs"][ci] if d != 0xFFFFFFFF else None)[:2]
        out = []
        for l in range(lanes):
            P = rows - 1
            out.append(O.accept_chain(P, rows, True, inp[l * rows + 1:(l + 1) * rows],
                                      vt[l * rows:(l + 1) * rows],
                                      cand_ids=c["cand_ids"][l * P:(l + 1) * P],
                                      cand_probs=c["cand_probs"][l * P:(l + 1) * P],
                                      target_draft_prob=vp[l * rows:(l + 1) * rows],
                                      uniforms40=c["uniforms"][l]))
        return vt, vp, out

    n, t0 = 0, time.perf_counter()
    while True:
        step()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds and n >= 2:
            break
    return dict(value=n / el, unit="steps/s", cores=1, kind="port", cpu_model=cpu_model(),
                sample=f"{n} whole verify steps ({lanes * rows} rows' selections with extras "
                       f"and sparse drafts, then {lanes} lanes' chain acceptance) of the same "
                       f"seeded inputs in {el:.1f} s: oracle/jf_oracle.c -O2 through ctypes, "
                       f"one thread")


def bench_verify(args):
    """The penalized chain-verify shape (VerifyStep): its step timed from
    C++ as the sample path's is, its dominant kernel (the single pass with
    the verify rows' extra penalty tokens, select_fast_kernel<0, true, FastRows, NoFinish>)
    timed alone."""
    import torch
    from jf_sampler import workloads as WL
    c = WL.config_verify()
    g = VerifyStep(c)
    print(f"# {g.w['name']}: {len(g.copies)} rotated copies", file=sys.stderr, flush=True)
    for i in range(args.warmup):
        g.step(i)
    torch.cuda.synchronize()
    K = args.steps
    wall0 = time.perf_counter()
    cpp = time_cpp_loop(g, K, False)
    wall = time.perf_counter() - wall0
    ms_per_step = cpp["us_per_step"] / 1000.0
    batch = pick_batch(K)
    per = time_cpp_loop(g, K, False, batch=batch)["batch_us"].astype(np.float64)
    sel_mean, sel_p50 = time_select(g, args.warmup + K, K)
    B, V = g.w["rows"], g.w["V"]
    H = len(c["histories"][0])
    # Algorithmic bytes of the selection kernel: every row's logits, its
    # lane's history ids (each row applies them), its extra tokens and its
    # 16 candidates; the step adds uniforms, outputs and the acceptance.
    sel_bytes = B * V * 4 + B * H * 4 + int(np.sum(c["extra_counts"])) * 4 + B * 16 * 8
    step_bytes = sel_bytes + B * 4 * 3 + c["lanes"] * (c["rows"] - 1) * (4 + 16 * 8)
    achieved = sel_bytes / (sel_mean * 1e-6) / 1e9
    step_gbs = step_bytes / (cpp["us_per_step"] * 1e-6) / 1e9
    kernel = "jf::select_fast_kernel<0, true, jf::FastRows, jf::NoFinish>"
    key = ("verify", "auto")
    traffic = read_traffic(key, kernel)
    prof_us = read_profile_us(key, kernel)
    cpu = None if args.no_cpu else verify_cpu_baseline(c, args.cpu_seconds)
    line = {
        "metric": "verify steps/sec at 4 lanes x 16 rows, V=248320 (select + chain "
                  "acceptance); achieved HBM GB/s vs peak; p50 us/step",
        "value": 1000.0 / ms_per_step, "unit": "steps/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": ms_per_step,
        "p50_us": float(np.percentile(per, 50)), "p90_us": float(np.percentile(per, 90)),
        "wall_s": wall, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (workloads.config_verify, seed 8), {len(g.copies)} rotated "
                f"logits copies >= 512 MB",
        "config": {"workload": g.w["name"], "rows": B, "vocabulary": V,
                   "algorithmic_bytes_per_step": step_bytes},
        "timing": f"jf_sample + jf_accept_chain back to back from C++, events at the loop's "
                  f"two ends; p50/p90 over runs of {batch} steps in a second pass",
        "host_us_per_call": cpp["host_us_per_call"],
        "host_issue_us": host_issue_us(g),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic, "kernel": kernel,
                     "timing": "mean of HIP events the library records around the kernel's "
                               "launch on its stream",
                     "kernel_mean_us": sel_mean, "kernel_p50_us": sel_p50,
                     "rocprof_mean_us": prof_us,
                     "rocprof_frac": (sel_bytes / (prof_us * 1e-6) / 1e9 / PEAK_HBM_GBS
                                      if prof_us else None),
                     "algorithmic_bytes": sel_bytes, "step_achieved": step_gbs,
                     "step_frac": step_gbs / PEAK_HBM_GBS},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    g.close()


def main():
    args = parse()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: every box has one "
                          "MI355X, and rows would shard across GPUs with no "
                          "exchange (each GPU samples its own rows), so run "
                          "--gpus 1"}))
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    if args.path == "draft":
        bench_draft(args)
        return
    if args.path == "gather":
        bench_gather(args)
        return
    if args.path == "verify":
        bench_verify(args)
        return
    if args.history != "uniform" and args.config != 2:
        print("--history applies to --config 2 only", file=sys.stderr)
        sys.exit(2)
    w = build_workload(args.config, args.mode, args.history)
    print(f"# {w['name']}: building inputs", file=sys.stderr, flush=True)
    # Table rows hold room for the counted loop's tokens and its warm-up's.
    count_warm = max(args.warmup, 32)
    g = GpuStep(w, count_headroom=args.steps + count_warm)
    for i in range(args.warmup):
        g.step(i)
    torch.cuda.synchronize()
    K = args.steps
    # The timed steps: jf_sample issued back to back from C++ (the engine's
    # call), HIP events on the launch stream at the loop's two ends only, a
    # device synchronization on both sides: `value`. Then a second pass of
    # K steps with an event after every `batch` steps for the distribution
    # (p50/p90 over those runs' mean step times): an event between steps
    # adds its own packets to the steps around it.
    wall0 = time.perf_counter()
    cpp = time_cpp_loop(g, K, False)
    wall = time.perf_counter() - wall0
    ms_per_step = cpp["us_per_step"] / 1000.0
    batch = pick_batch(K)
    per = time_cpp_loop(g, K, False, batch=batch)["batch_us"].astype(np.float64)
    p50, p90 = float(np.percentile(per, 50)), float(np.percentile(per, 90))
    step_gbs = w["alg_bytes"] / (cpp["us_per_step"] * 1e-6) / 1e9
    # The same steps from a Python loop (ctypes per call), for comparison.
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(K):
        g.step(args.warmup + i)
        ev[i + 1].record()
    torch.cuda.synchronize()
    py_per = np.array([ev[i].elapsed_time(ev[i + 1]) for i in range(K)]) * 1000.0
    python_loop = {"ms_per_step": ev[0].elapsed_time(ev[K]) / K,
                   "p50_us": float(np.percentile(py_per, 50))}
    # The dominant kernel (the single pass over the logits) timed alone; its
    # algorithmic bytes are the logits and the history ids or mask words.
    sel_mean, sel_p50 = time_select(g, args.warmup + K, K)
    achieved = w["select_bytes"] / (sel_mean * 1e-6) / 1e9
    graphed = time_graph(g, K)
    counted = None
    if g.tables:
        # Warm-up first, untimed: every rotated copy's table takes its first
        # counts (host copy growth, first touches) here. Each table then
        # takes at most (warm + K) / tables + 1 <= K + count_warm tokens a
        # row, the headroom its rows were given.
        time_cpp_loop(g, max(count_warm, len(g.tables)), True)
        counted = time_cpp_loop(g, K, True)
        counted["note"] = ("each step followed by jf_penalty_table_count_rows of one "
                           "token per row, from C++")
    cpu = None if args.no_cpu else cpu_baseline(w, args.cpu_seconds)
    # Every benchmarked sample workload is a uniform launch (one policy, each
    # row its own penalty row): the fast kernel's variant without per-row facts.
    kernel = w.get("kernel",
                   f"jf::select_fast_kernel<{0 if w['dtype'] == 'f32' else 1}, false, jf::NoRows, "
                   "jf::NoFinish>")
    key = profile_key(args.config, args.mode, args.history)
    traffic = read_traffic(key, kernel)
    prof_us = read_profile_us(key, kernel)
    line = {
        "metric": "sampling steps/sec at B=64,V=151936; achieved HBM GB/s vs peak; p50 us/step",
        "value": 1000.0 / ms_per_step,
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "p50_us": p50,
        "p90_us": p90,
        "wall_s": wall,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w["dtype"],
        "data": f"synthetic (seeded generators in justfit-llm_amd/jf_sampler/workloads.py), "
                f"{len(g.copies)} rotated input copies >= 512 MB",
        "config": {"workload": w["name"], "rows": w["rows"], "vocabulary": w["V"],
                   "algorithmic_bytes_per_step": w["alg_bytes"]},
        "timing": "jf_sample called back to back from C++ (libjf_bench_loop.so), HIP events "
                  "on the launch stream at the loop's two ends (value, ms_per_step); p50/p90 "
                  f"over the runs of a second pass of {K} steps with an event every {batch} "
                  "steps; host_us_per_call is the first loop's own issue time (paced by the "
                  "GPU once the device queue is full); host_issue_us is the median host cost "
                  "of a step in 16-step bursts issued to an idle stream",
        "host_us_per_call": cpp["host_us_per_call"],
        "host_issue_us": host_issue_us(g),
        "python_loop": python_loop,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": achieved / PEAK_HBM_GBS,
                     "traffic": traffic,
                     "kernel": kernel,
                     "timing": "mean of HIP events the library records around the kernel's "
                               "launch (hipExtLaunchKernelGGL) on its stream",
                     "kernel_mean_us": sel_mean, "kernel_p50_us": sel_p50,
                     "rocprof_mean_us": prof_us,
                     "rocprof_frac": (w["select_bytes"] / (prof_us * 1e-6) / 1e9 / PEAK_HBM_GBS
                                      if prof_us else None),
                     "algorithmic_bytes": w["select_bytes"],
                     "step_achieved": step_gbs,
                     "step_frac": step_gbs / PEAK_HBM_GBS},
        "with_penalty_count": counted,
        "graph_replay": graphed,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
