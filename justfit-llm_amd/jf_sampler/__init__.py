"""ctypes binding of libjf_sampler.so (the C ABI in include/jf_sampler.h).

Tests and bench.py drive the HIP sampler through this module. Device memory
comes from torch tensors (plumbing only): every pointer handed to the library
is a tensor's data_ptr(), and work is enqueued on torch's current HIP stream.
The module refuses to run without the built library; there is no fallback.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libjf_sampler.so")

JF_OK = 0
JF_ERR_INVALID_ARGUMENT = 1
JF_ERR_LOGIC = 2
JF_ERR_DEVICE = 3
JF_NO_TOKEN = 0xFFFFFFFF
JF_DTYPE_F32 = 0
JF_DTYPE_BF16 = 1
JF_POLICY_CONSTRAINED = 1
JF_POLICY_EXCLUDE_STOP = 2
JF_SAMPLING_UNIFORMS = 40
JF_DRAFT_CANDIDATES = 16
JF_UNIFORM_ACCEPTANCE = 8
JF_UNIFORM_CORRECTION = 15
JF_UNIFORM_TREE_DRAWS = 24

# Every symbol include/jf_sampler.h declares.
EXPORTS = [
    "jf_last_error", "jf_policy_validate", "jf_sampler_create",
    "jf_sampler_destroy", "jf_sampler_workspace_bytes", "jf_sampler_status",
    "jf_sampler_set_wait_bound",
    "jf_penalty_words_rebuild", "jf_penalty_words_count",
    "jf_penalty_table_create", "jf_penalty_table_destroy",
    "jf_penalty_table_rebuild", "jf_penalty_table_count", "jf_penalty_table_count_rows",
    "jf_next_uniform", "jf_stage_sampling_cycle", "jf_sample", "jf_sample_static",
    "jf_accept_chain", "jf_accept_tree", "jf_sample_accept_tree",
    "jf_draft_selector_create", "jf_draft_selector_destroy", "jf_draft_select",
    "jf_tree_gather", "jf_build_draft_tree", "jf_mask_request_encode",
    "jf_mask_response_decode", "jf_mask_rows_check", "jf_mask_chain_fill", "jf_mask_tree_fill",
]

c_u32 = ctypes.c_uint32
c_u64 = ctypes.c_uint64
c_f32 = ctypes.c_float
c_vp = ctypes.c_void_p


class JfPolicy(ctypes.Structure):
    _fields_ = [("top_k", c_u32), ("temperature", c_f32), ("top_p", c_f32),
                ("min_p", c_f32), ("repetition", c_f32), ("presence", c_f32),
                ("frequency", c_f32), ("flags", c_u32)]


class JfSampleArgs(ctypes.Structure):
    _fields_ = [
        ("rows", c_u32), ("dtype", c_u32), ("logits", c_vp),
        ("logits_stride", c_u64), ("masks", c_vp), ("mask_stride", c_u64),
        ("policies", ctypes.POINTER(JfPolicy)), ("stop_token_0", c_u32),
        ("stop_token_1", c_u32), ("penalties", c_vp),
        ("penalty_rows", ctypes.POINTER(c_u32)), ("extra_tokens", c_vp),
        ("extra_counts", ctypes.POINTER(c_u32)), ("extra_stride", c_u64),
        ("uniforms", c_vp), ("uniform_index", c_vp), ("uniform_offset", c_u64),
        ("uniform_stride", c_u64), ("draft_tokens", c_vp),
        ("drafted_rows", c_u32), ("draft_cand_ids", c_vp),
        ("draft_cand_probs", c_vp), ("draft_q", c_vp),
        ("draft_q_stride", c_u64), ("out_tokens", c_vp),
        ("out_draft_probs", c_vp), ("out_kept_counts", c_vp),
        ("out_kept_ids", c_vp), ("out_kept_probs", c_vp),
        ("kept_capacity", c_u32), ("select_start_event", c_vp),
        ("select_done_event", c_vp), ("mask_rows", ctypes.POINTER(c_u32)),
        ("draft_token_index", ctypes.POINTER(c_u32)),
        ("draft_cand_index", ctypes.POINTER(c_u32)),
        ("extra_offsets", ctypes.POINTER(c_u64)),
    ]


class JfAcceptChainArgs(ctypes.Structure):
    _fields_ = [
        ("lanes", c_u32), ("verify_rows", c_u32), ("proposed_tokens", c_vp),
        ("candidates", c_vp), ("proposal_probs", c_vp),
        ("target_draft_probs", c_vp), ("uniforms", c_vp),
        ("target_tokens", c_vp), ("retained_counts", c_vp),
        ("accepted_counts", c_vp),
        ("maximum_retained", ctypes.POINTER(c_u32)),
        ("policies", ctypes.POINTER(JfPolicy)), ("stop_token_0", c_u32),
        ("stop_token_1", c_u32),
    ]


class JfTreeLane(ctypes.Structure):
    _fields_ = [("rows", c_u32), ("chain_rows", c_u32),
                ("parent", c_u32 * 16), ("token", c_u32 * 16),
                ("chain_q", c_f32 * 8)]


class JfAcceptTreeArgs(ctypes.Structure):
    _fields_ = [
        ("lanes", c_u32), ("rows_per_lane", c_u32),
        ("trees", ctypes.POINTER(JfTreeLane)), ("target_draft_probs", c_vp),
        ("uniforms", c_vp), ("target_tokens", c_vp),
        ("retained_counts", c_vp), ("accepted_counts", c_vp),
        ("path_rows", c_vp), ("maximum_retained", ctypes.POINTER(c_u32)),
        ("policies", ctypes.POINTER(JfPolicy)), ("stop_token_0", c_u32),
        ("stop_token_1", c_u32),
    ]


class JfDraftSelectArgs(ctypes.Structure):
    _fields_ = [
        ("lanes", c_u32), ("logits", c_vp), ("logits_stride", c_u64),
        ("selector_hidden", c_vp), ("predecessor_codebook", c_vp),
        ("successor_codebook", c_vp), ("anchors", c_vp), ("policies", c_vp),
        ("uniforms", c_vp), ("candidates", c_vp), ("unary", c_vp),
        ("proposed_tokens", c_vp), ("proposal_probs", c_vp),
        ("select_start_event", c_vp), ("select_done_event", c_vp),
        ("edge_tables", c_vp),
    ]


class JfTreeGatherArgs(ctypes.Structure):
    _fields_ = [("data", c_vp), ("data_units", c_u64), ("path_rows", c_vp), ("retained", c_vp)] + [
        (n, c_u32) for n in ("columns", "inner", "inner_stride", "outer_stride", "row_stride",
                             "lane_stride", "layer_stride", "layers", "lanes", "rows")] + [
        ("start_event", c_vp), ("done_event", c_vp)]


class JfDraftTree(ctypes.Structure):
    _fields_ = [("rows", c_u32), ("copies", c_u32), ("parent", c_u32 * 16), ("depth", c_u32 * 16),
                ("copy", c_u32 * 16), ("token", c_u32 * 16), ("path_length", c_u32 * 16),
                ("path", (c_u32 * 8) * 16)]


class JfError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(f"jf error {code}: {message}")
        self.code = code
        self.message = message


_lib = None


def lib():
    """The loaded library; raises if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with "
                "python justfit-llm_amd/build.py (no fallback exists)")
        # One HIP runtime per process: torch's, which owns the device memory
        # and streams handed to the library. Loaded first, its
        # libamdhip64.so.7 is the one the library's dependency resolves to
        # (loaded after the library, torch would bring a second runtime), and
        # it is initialized before the library registers its code objects.
        import torch
        torch.cuda.is_available()
        L = ctypes.CDLL(LIB_PATH)
        L.jf_last_error.restype = ctypes.c_char_p
        L.jf_policy_validate.argtypes = [ctypes.POINTER(JfPolicy)]
        L.jf_sampler_create.argtypes = [c_u32, c_u32, ctypes.POINTER(c_vp)]
        L.jf_sampler_destroy.argtypes = [c_vp]
        L.jf_sampler_workspace_bytes.argtypes = [c_vp]
        L.jf_sampler_workspace_bytes.restype = c_u64
        L.jf_sampler_status.argtypes = [c_vp, c_vp]
        L.jf_sampler_set_wait_bound.argtypes = [c_vp, c_u32]
        L.jf_penalty_words_rebuild.argtypes = [
            c_vp, c_u32, c_vp, c_u64, c_u64, ctypes.c_int, c_u32, ctypes.c_int]
        L.jf_penalty_words_count.argtypes = [c_vp, c_u32, c_vp, c_u64]
        L.jf_penalty_table_create.argtypes = [c_u32, c_u32, c_u32,
                                              ctypes.POINTER(c_vp)]
        L.jf_penalty_table_destroy.argtypes = [c_vp]
        L.jf_penalty_table_rebuild.argtypes = [
            c_vp, c_u32, c_vp, c_u64, c_u64, ctypes.c_int, c_u32,
            ctypes.c_int, c_vp]
        L.jf_penalty_table_count.argtypes = [c_vp, c_u32, c_vp, c_u64, c_vp]
        L.jf_penalty_table_count_rows.argtypes = [c_vp, c_vp, c_vp, c_u64, c_vp]
        L.jf_next_uniform.argtypes = [c_u64, ctypes.POINTER(c_u64)]
        L.jf_next_uniform.restype = c_f32
        L.jf_stage_sampling_cycle.argtypes = [
            c_u64, ctypes.POINTER(c_u64), c_u32, ctypes.c_int, c_vp]
        L.jf_stage_sampling_cycle.restype = None
        L.jf_sample.argtypes = [c_vp, ctypes.POINTER(JfSampleArgs), c_vp]
        L.jf_sample_static.argtypes = [c_u32, ctypes.POINTER(JfSampleArgs), c_vp]
        L.jf_accept_chain.argtypes = [c_vp, ctypes.POINTER(JfAcceptChainArgs),
                                      c_vp]
        L.jf_accept_tree.argtypes = [c_vp, ctypes.POINTER(JfAcceptTreeArgs),
                                     c_vp]
        L.jf_sample_accept_tree.argtypes = [c_vp, ctypes.POINTER(JfSampleArgs),
                                            ctypes.POINTER(JfAcceptTreeArgs), c_vp]
        L.jf_draft_selector_create.argtypes = [c_u32, c_u32, ctypes.POINTER(c_vp)]
        L.jf_draft_selector_destroy.argtypes = [c_vp]
        L.jf_draft_select.argtypes = [c_vp, ctypes.POINTER(JfDraftSelectArgs), c_vp]
        L.jf_tree_gather.argtypes = [ctypes.POINTER(JfTreeGatherArgs), c_vp]
        L.jf_build_draft_tree.argtypes = [c_vp, c_vp, c_vp, c_u32, c_u32, c_vp,
                                          ctypes.POINTER(JfDraftTree), ctypes.POINTER(ctypes.c_double),
                                          ctypes.POINTER(ctypes.c_double)]
        L.jf_mask_request_encode.argtypes = [c_u64, c_u64, c_u32, c_vp, c_u32, c_vp, c_vp, c_u64,
                                             ctypes.POINTER(c_u64)]
        L.jf_mask_response_decode.argtypes = [c_vp, c_u64, ctypes.POINTER(c_u64),
                                              ctypes.POINTER(c_u64), c_vp, c_u32,
                                              ctypes.POINTER(c_u32)]
        L.jf_mask_rows_check.argtypes = [c_vp, c_u32, c_u32, c_u32]
        L.jf_mask_chain_fill.argtypes = [c_vp, c_u32, c_u32, c_u32]
        L.jf_mask_tree_fill.argtypes = [c_vp, c_u32, c_vp, c_vp, c_u32]
        _lib = L
    return _lib


def check(rc):
    if rc != JF_OK:
        raise JfError(rc, lib().jf_last_error().decode())


def sample_static(vocabulary, a, stream=None):
    """jf_sample_static: one selection with the library's static device
    scratch (no sampler object, no allocation); `a` as Sampler.sample_args
    builds it."""
    check(lib().jf_sample_static(vocabulary, ctypes.byref(a),
                                 _stream() if stream is None else stream))


def policy(top_k=0, temperature=0.0, top_p=1.0, min_p=0.0, repetition=1.0,
           presence=0.0, frequency=0.0, constrained=False, exclude_stop=False):
    """A jf_policy with the reference request defaults (greedy, neutral)."""
    flags = (JF_POLICY_CONSTRAINED if constrained else 0) | (
        JF_POLICY_EXCLUDE_STOP if exclude_stop else 0)
    return JfPolicy(top_k, temperature, top_p, min_p, repetition, presence,
                    frequency, flags)


def validate(p):
    check(lib().jf_policy_validate(ctypes.byref(p)))


def next_uniform(seed, counter):
    """(uniform, new counter): Runtime::nextUniform."""
    c = c_u64(counter)
    u = lib().jf_next_uniform(seed, ctypes.byref(c))
    return u, c.value


def stage_cycle(seed, counter, verify_rows, tree_cycle):
    import numpy as np
    out = np.zeros(40, dtype=np.float32)
    c = c_u64(counter)
    lib().jf_stage_sampling_cycle(seed, ctypes.byref(c), verify_rows,
                                  1 if tree_cycle else 0,
                                  out.ctypes.data_as(c_vp))
    return out, c.value


def rebuild_penalty_words(words, history, generated, pending, mark_prompt):
    """Dense host words (numpy uint32[V]) as Sampling::rebuildPenaltyWords."""
    import numpy as np
    h = np.ascontiguousarray(history, dtype=np.uint32)
    check(lib().jf_penalty_words_rebuild(
        words.ctypes.data_as(c_vp), words.size, h.ctypes.data_as(c_vp),
        h.size, generated, 0 if pending is None else 1,
        0 if pending is None else pending, 1 if mark_prompt else 0))


def count_penalty_tokens(words, selected):
    import numpy as np
    s = np.ascontiguousarray(selected, dtype=np.uint32)
    check(lib().jf_penalty_words_count(words.ctypes.data_as(c_vp), words.size,
                                       s.ctypes.data_as(c_vp), s.size))


def _stream():
    import torch
    return c_vp(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return None if t is None else c_vp(t.data_ptr())


class PenaltyTable:
    """jf_penalty_table: sparse device penalty words, one row per state lane."""

    def __init__(self, vocabulary, rows, max_entries):
        h = c_vp()
        check(lib().jf_penalty_table_create(vocabulary, rows, max_entries,
                                            ctypes.byref(h)))
        self.handle = h
        self.vocabulary = vocabulary
        self.rows = rows

    def rebuild(self, row, history, generated, pending=None, mark_prompt=False):
        import numpy as np
        h = np.ascontiguousarray(history, dtype=np.uint32)
        check(lib().jf_penalty_table_rebuild(
            self.handle, row, h.ctypes.data_as(c_vp), h.size, generated,
            0 if pending is None else 1, 0 if pending is None else pending,
            1 if mark_prompt else 0, _stream()))

    def count(self, row, selected):
        import numpy as np
        s = np.ascontiguousarray(selected, dtype=np.uint32)
        check(lib().jf_penalty_table_count(self.handle, row,
                                           s.ctypes.data_as(c_vp), s.size,
                                           _stream()))

    def count_rows(self, rows, selected):
        """One step's commits of several rows: token selected[i] into row rows[i]."""
        import numpy as np
        r = np.ascontiguousarray(rows, dtype=np.uint32)
        s = np.ascontiguousarray(selected, dtype=np.uint32)
        if r.size != s.size:
            raise ValueError("rows and selected differ in length")
        check(lib().jf_penalty_table_count_rows(self.handle, r.ctypes.data_as(c_vp),
                                                s.ctypes.data_as(c_vp), s.size, _stream()))

    def close(self):
        if self.handle:
            lib().jf_penalty_table_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sampler:
    """jf_sampler: one vocabulary, up to max_rows selected rows per call."""

    def __init__(self, vocabulary, max_rows):
        h = c_vp()
        check(lib().jf_sampler_create(vocabulary, max_rows, ctypes.byref(h)))
        self.handle = h
        self.vocabulary = vocabulary
        self.max_rows = max_rows

    def workspace_bytes(self):
        return lib().jf_sampler_workspace_bytes(self.handle)

    def status(self, stream=None):
        """jf_sampler_status: raises JfError (JF_ERR_DEVICE) once if a greedy
        finisher's bounded wait expired in a call that has run."""
        check(lib().jf_sampler_status(self.handle, _stream() if stream is None else stream))

    def set_wait_bound(self, reads):
        check(lib().jf_sampler_set_wait_bound(self.handle, reads))

    def sample_args(self, logits, policies, out_tokens, *, masks=None,
                    stop_tokens=(JF_NO_TOKEN, JF_NO_TOKEN), penalties=None,
                    penalty_rows=None, extra_tokens=None, extra_counts=None,
                    extra_stride=0, uniforms=None, uniform_index=None,
                    uniform_offset=0, uniform_stride=1, draft_tokens=None,
                    drafted_rows=None, cand_ids=None, cand_probs=None,
                    dense_q=None, out_draft_probs=None, kept=None, mask_rows=None,
                    draft_token_index=None, draft_cand_index=None, extra_offsets=None):
        """Builds a JfSampleArgs (kept-alive host arrays ride along)."""
        import torch
        rows = logits.shape[0]
        a = JfSampleArgs()
        a.rows = rows
        a.dtype = JF_DTYPE_BF16 if logits.dtype == torch.bfloat16 else JF_DTYPE_F32
        a.logits = logits.data_ptr()
        a.logits_stride = logits.stride(0)
        if masks is not None:
            a.masks = masks.data_ptr()
            a.mask_stride = masks.stride(0)
        pol = (JfPolicy * rows)(*policies)
        a.policies = pol
        a.stop_token_0, a.stop_token_1 = stop_tokens
        keep = [pol]
        if penalties is not None:
            a.penalties = penalties.handle
            pr = (c_u32 * rows)(*penalty_rows)
            a.penalty_rows = pr
            keep.append(pr)
        if extra_tokens is not None:
            a.extra_tokens = extra_tokens.data_ptr()
            ec = (c_u32 * rows)(*extra_counts)
            a.extra_counts = ec
            a.extra_stride = extra_stride
            keep.append(ec)
        if uniforms is not None:
            a.uniforms = uniforms.data_ptr()
        if uniform_index is not None:
            a.uniform_index = uniform_index.data_ptr()
        a.uniform_offset = uniform_offset
        a.uniform_stride = uniform_stride
        if draft_tokens is not None:
            a.draft_tokens = draft_tokens.data_ptr()
            a.drafted_rows = rows if drafted_rows is None else drafted_rows
        if cand_ids is not None:
            a.draft_cand_ids = cand_ids.data_ptr()
            a.draft_cand_probs = cand_probs.data_ptr()
        if dense_q is not None:
            a.draft_q = dense_q.data_ptr()
            a.draft_q_stride = dense_q.stride(0)
        a.out_tokens = out_tokens.data_ptr()
        if out_draft_probs is not None:
            a.out_draft_probs = out_draft_probs.data_ptr()
        if kept is not None:
            counts, ids, probs = kept
            a.out_kept_counts = counts.data_ptr()
            a.out_kept_ids = ids.data_ptr()
            a.out_kept_probs = probs.data_ptr()
            a.kept_capacity = ids.shape[1]
        for name, values, ctype in (("mask_rows", mask_rows, c_u32),
                                    ("draft_token_index", draft_token_index, c_u32),
                                    ("draft_cand_index", draft_cand_index, c_u32),
                                    ("extra_offsets", extra_offsets, c_u64)):
            if values is not None:
                arr = (ctype * rows)(*[int(v) for v in values])
                setattr(a, name, arr)
                keep.append(arr)
        return a, keep

    def sample(self, *args, **kwargs):
        a, keep = self.sample_args(*args, **kwargs)
        self.launch(a)
        return keep

    def launch(self, a, stream=None):
        check(lib().jf_sample(self.handle, ctypes.byref(a),
                              _stream() if stream is None else stream))

    def accept_chain_args(self, *, verify_rows, proposed, target_tokens, retained,
                          accepted, maximum_retained, policies, candidates=None,
                          proposal_probs=None, target_draft_probs=None,
                          uniforms=None, stop_tokens=(JF_NO_TOKEN, JF_NO_TOKEN)):
        """Builds a JfAcceptChainArgs (kept-alive host arrays ride along)."""
        lanes = len(maximum_retained)
        a = JfAcceptChainArgs()
        a.lanes = lanes
        a.verify_rows = verify_rows
        a.proposed_tokens = proposed.data_ptr()
        a.candidates = None if candidates is None else candidates.data_ptr()
        a.proposal_probs = None if proposal_probs is None else proposal_probs.data_ptr()
        a.target_draft_probs = (None if target_draft_probs is None
                                else target_draft_probs.data_ptr())
        a.uniforms = None if uniforms is None else uniforms.data_ptr()
        a.target_tokens = target_tokens.data_ptr()
        a.retained_counts = retained.data_ptr()
        a.accepted_counts = accepted.data_ptr()
        mr = (c_u32 * lanes)(*maximum_retained)
        pol = (JfPolicy * lanes)(*policies)
        a.maximum_retained = mr
        a.policies = pol
        a.stop_token_0, a.stop_token_1 = stop_tokens
        return a, [mr, pol]

    def launch_accept(self, acc, stream=None):
        """Issues a prepared acceptance: ("chain" | "tree", args, keep)."""
        fn = lib().jf_accept_chain if acc[0] == "chain" else lib().jf_accept_tree
        check(fn(self.handle, ctypes.byref(acc[1]), _stream() if stream is None else stream))

    def accept_chain(self, **kwargs):
        a, keep = self.accept_chain_args(**kwargs)
        check(lib().jf_accept_chain(self.handle, ctypes.byref(a), _stream()))

    def accept_tree_args(self, *, trees, rows_per_lane, target_tokens, retained,
                         accepted, path_rows, maximum_retained, policies,
                         target_draft_probs=None, uniforms=None,
                         stop_tokens=(JF_NO_TOKEN, JF_NO_TOKEN)):
        """Builds a JfAcceptTreeArgs (kept-alive host arrays ride along)."""
        lanes = len(trees)
        a = JfAcceptTreeArgs()
        a.lanes = lanes
        a.rows_per_lane = rows_per_lane
        tl = (JfTreeLane * lanes)(*trees)
        a.trees = tl
        a.target_draft_probs = (None if target_draft_probs is None
                                else target_draft_probs.data_ptr())
        a.uniforms = None if uniforms is None else uniforms.data_ptr()
        a.target_tokens = target_tokens.data_ptr()
        a.retained_counts = retained.data_ptr()
        a.accepted_counts = accepted.data_ptr()
        a.path_rows = path_rows.data_ptr()
        mr = (c_u32 * lanes)(*maximum_retained)
        pol = (JfPolicy * lanes)(*policies)
        a.maximum_retained = mr
        a.policies = pol
        a.stop_token_0, a.stop_token_1 = stop_tokens
        return a, [tl, mr, pol]

    def accept_tree(self, **kwargs):
        a, keep = self.accept_tree_args(**kwargs)
        check(lib().jf_accept_tree(self.handle, ctypes.byref(a), _stream()))

    def launch_sample_accept_tree(self, sample_args, tree_args, stream=None):
        """jf_sample_accept_tree over prepared JfSampleArgs and JfAcceptTreeArgs."""
        check(lib().jf_sample_accept_tree(self.handle, ctypes.byref(sample_args),
                                          ctypes.byref(tree_args),
                                          _stream() if stream is None else stream))

    def close(self):
        if self.handle:
            lib().jf_sampler_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DraftSelector:
    """jf_draft_selector: the DFlash draft's proposal policy for up to
    max_lanes lanes (ops::DraftSelector)."""

    def __init__(self, vocabulary, max_lanes):
        h = c_vp()
        check(lib().jf_draft_selector_create(vocabulary, max_lanes, ctypes.byref(h)))
        self.handle = h
        self.vocabulary = vocabulary
        self.max_lanes = max_lanes

    def args(self, *, logits, hidden, pred_codebook, succ_codebook, anchors, policies,
             candidates, unary, tokens, q=None, uniforms=None, stride=None, edge_tables=None):
        """A jf_draft_select_args over torch device tensors; `anchors` and
        `policies` are host sequences (kept alive on the returned object)."""
        import numpy as np
        lanes = len(anchors)
        a = JfDraftSelectArgs()
        a.lanes = lanes
        a.logits = _ptr(logits)
        a.logits_stride = stride if stride is not None else logits.shape[-1]
        a.selector_hidden = _ptr(hidden)
        a.predecessor_codebook = _ptr(pred_codebook)
        a.successor_codebook = _ptr(succ_codebook)
        anc = np.ascontiguousarray(anchors, dtype=np.uint32)
        pol = (JfPolicy * lanes)(*policies)
        a.anchors = anc.ctypes.data_as(c_vp)
        a.policies = ctypes.cast(pol, c_vp)
        a.uniforms = _ptr(uniforms)
        a.candidates = _ptr(candidates)
        a.unary = _ptr(unary)
        a.proposed_tokens = _ptr(tokens)
        a.proposal_probs = _ptr(q)
        a.edge_tables = _ptr(edge_tables)
        a._keep = (anc, pol)
        return a

    def launch(self, a, stream=None):
        check(lib().jf_draft_select(self.handle, ctypes.byref(a),
                                    stream if stream is not None else _stream()))

    def close(self):
        if self.handle:
            lib().jf_draft_selector_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def tree_gather_args(data, path_rows, retained, **layout):
    """A jf_tree_gather_args over torch device tensors (data: 16-bit
    elements); layout: columns, inner, inner_stride, outer_stride,
    row_stride, lane_stride, layer_stride, layers, lanes, rows."""
    a = JfTreeGatherArgs()
    a.data = _ptr(data)
    a.data_units = data.numel()
    a.path_rows = _ptr(path_rows)
    a.retained = _ptr(retained)
    for k, v in layout.items():
        setattr(a, k, v)
    return a


def tree_gather(a, stream=None):
    check(lib().jf_tree_gather(ctypes.byref(a), stream if stream is not None else _stream()))


def build_draft_tree(candidates, unary, edges, anchor, rows, chain_picks=None):
    """jf_build_draft_tree on host arrays; returns the tree as a dict plus
    expected / chain_expected."""
    import numpy as np
    c = np.ascontiguousarray(candidates, dtype=np.uint32)
    u = np.ascontiguousarray(unary, dtype=np.float32)
    e = np.ascontiguousarray(edges, dtype=np.float32)
    cp = None if chain_picks is None else np.ascontiguousarray(chain_picks, dtype=np.uint32)
    t = JfDraftTree()
    ex, cx = ctypes.c_double(), ctypes.c_double()
    check(lib().jf_build_draft_tree(c.ctypes.data_as(c_vp), u.ctypes.data_as(c_vp),
                                    e.ctypes.data_as(c_vp), anchor, rows,
                                    None if cp is None else cp.ctypes.data_as(c_vp),
                                    ctypes.byref(t), ctypes.byref(ex), ctypes.byref(cx)))
    return dict(rows=t.rows, copies=t.copies, parent=list(t.parent), depth=list(t.depth),
                copy=list(t.copy), token=list(t.token), path_length=list(t.path_length),
                path=[list(r) for r in t.path], expected=ex.value, chain_expected=cx.value)


def mask_request_encode(request_id, mask_id, words_per_mask, tokens, parents=None):
    """One MaskRequest (or, with parents, MaskTreeRequest) frame as bytes."""
    import numpy as np
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    p = None if parents is None else np.ascontiguousarray(parents, dtype=np.uint32)
    out = np.zeros(16 + 24 + 8 * len(t), np.uint8)
    n = c_u64()
    check(lib().jf_mask_request_encode(request_id, mask_id, words_per_mask,
                                       t.ctypes.data_as(c_vp), len(t),
                                       None if p is None else p.ctypes.data_as(c_vp),
                                       out.ctypes.data_as(c_vp), out.size, ctypes.byref(n)))
    return out[:n.value].tobytes()


def mask_response_decode(frame, capacity=1 << 20):
    """(request_id, mask_request_id, words) of one MaskResponse frame."""
    import numpy as np
    f = np.frombuffer(frame, dtype=np.uint8)
    words = np.zeros(capacity, np.uint32)
    rid, mid, n = c_u64(), c_u64(), c_u32()
    check(lib().jf_mask_response_decode(f.ctypes.data_as(c_vp), f.size, ctypes.byref(rid),
                                        ctypes.byref(mid), words.ctypes.data_as(c_vp), capacity,
                                        ctypes.byref(n)))
    return rid.value, mid.value, words[:n.value].copy()


def mask_rows_check(words, rows, mask_words, pending_token=JF_NO_TOKEN):
    import numpy as np
    w = np.ascontiguousarray(words, dtype=np.uint32)
    check(lib().jf_mask_rows_check(w.ctypes.data_as(c_vp), rows, mask_words, pending_token))


def mask_chain_fill(words, count, valid, mask_words):
    import numpy as np
    w = np.ascontiguousarray(words, dtype=np.uint32).copy()
    check(lib().jf_mask_chain_fill(w.ctypes.data_as(c_vp), count, valid, mask_words))
    return w


def mask_tree_fill(words, parents, refused, mask_words):
    import numpy as np
    w = np.ascontiguousarray(words, dtype=np.uint32).copy()
    p = np.ascontiguousarray(parents, dtype=np.uint32)
    r = np.ascontiguousarray(refused, dtype=np.uint8)
    check(lib().jf_mask_tree_fill(w.ctypes.data_as(c_vp), len(p), p.ctypes.data_as(c_vp),
                                  r.ctypes.data_as(c_vp), mask_words))
    return w


def tree_lane(parent, token, chain_rows=0, chain_q=None):
    t = JfTreeLane()
    t.rows = len(parent)
    t.chain_rows = chain_rows
    for i, p in enumerate(parent):
        t.parent[i] = p
    for i, tok in enumerate(token):
        t.token[i] = tok
    if chain_q is not None:
        for i, q in enumerate(chain_q):
            t.chain_q[i] = q
    return t
