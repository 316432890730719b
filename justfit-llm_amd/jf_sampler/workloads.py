"""Seeded synthetic inputs of the five benchmark configurations.

Each generator returns plain numpy arrays (host); callers move them to the
device. The formulas are fixed here so that tests, bench.py and the CPU
baseline see identical inputs:

C1 greedy      B=1, V=151,936 fp32 ~ N(0, 2^2) (seed 1); repetition 1.1 over
               a 256-token prompt of uniform ids.
C2 sampled     B=64, V=151,936 fp32 ~ N(0, 2.5^2) plus 8.0 at 8 distinct ids
               per row (seed 2); T 0.7, top-k 50, top-p 0.9, presence 0.5,
               frequency 0.3 over 2,048 generated ids (after a one-token
               prompt) per row; one SplitMix64
               uniform per row (seed row_seed(2, r), counter 1).
C3 grammar     B=32, V=151,936 bf16 ~ N(0, 2^2) (seed 3); packed mask: runs of
               U[1,40] tokens at uniform starts until >= 2% of V, plus 20
               single bits; greedy, and T 1.0 with nothing cut.
C4 tree        16 requests x 16-row DFS-preorder trees, branching U{1..3},
               depth <= 5, tokens U[0, V) (seed 4); target fp32 [256, V] ~
               N(0, 2^2); draft q per row = softmax(0.8 z + 0.6 e), z the
               standardized target row, e ~ N(0, 1); greedy and rejection
               acceptance (T 1.0, nothing cut).
C5 large       B=256, V=248,320 bf16 = 3 N(0,1) + t(3) (seed 5); repetition
               1.1, presence 0.5, frequency 0.3 over 8,192 ids (first 4,096
               prompt); min-p 0.05, top-k 1000, top-p 0.95, T 0.8.
verify         The engine's penalized chain verify (Sampling::addVerify,
               Sampling.cpp:149-172; penalize_verify, sampling.metal:978-993)
               at the reference's widest batch: 4 lanes x 16 verify rows of
               V=248,320 fp32 ~ N(0, 2.5^2) plus 8.0 at 8 ids per row (seed 8);
               each lane's 16 input tokens (the anchor, then 15 proposals,
               each proposal +14.0 in the row that verifies it); row r follows
               proposal r + 1 (rows 0..14) with 16 sparse candidates (0.6 on
               the proposal, Dirichlet(0.5) over the rest), counts
               the lane's proposals 1..r as extra penalty tokens, and draws
               with the lane's correction uniform (slot 15 of 40); T 0.7,
               top-k 50, top-p 0.9, repetition 1.1, presence 0.5, frequency
               0.3 over 2,048-id histories (the first 1,024 prompt); then
               chain acceptance (verify rows 16, all 16 retainable).
"""
import numpy as np

V_QWEN = 151936
V_LARGE = 248320
NO_TOKEN = 0xFFFFFFFF


def row_seed(config, row):
    return config * 1_000_003 + row


def splitmix_uniform(seed, counter):
    """Runtime::nextUniform for counter -> counter + 1 (the counter before)."""
    m = (1 << 64) - 1
    v = (seed + (counter + 1) * 0x9E3779B97F4A7C15) & m
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & m
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & m
    v ^= v >> 31
    return np.float32((v >> 40) * (2.0 ** -24))


def to_bf16_bits(x):
    """float32 -> bfloat16 bit patterns (round to nearest even)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return r.astype(np.uint16)


def bf16_bits_to_f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def mask_words(allowed_bool):
    """bool [rows, V] -> packed uint32 [rows, ceil(V/32)] (bit t%32 of word t/32)."""
    rows, V = allowed_bool.shape
    W = (V + 31) // 32
    pad = np.zeros((rows, W * 32), dtype=np.uint8)
    pad[:, :V] = allowed_bool
    bits = pad.reshape(rows, W, 32).astype(np.uint64)
    weights = (np.uint64(1) << np.arange(32, dtype=np.uint64))
    return (bits * weights).sum(axis=2).astype(np.uint32)


def config1(V=V_QWEN):
    rng = np.random.default_rng(1)
    logits = rng.normal(0.0, 2.0, (1, V)).astype(np.float32)
    history = rng.integers(0, V, 256, dtype=np.int64).astype(np.uint32)
    return dict(V=V, logits=logits, histories=[history], generated=[0],
                policy=dict(repetition=1.1), mark_prompt=True)


def config2(V=V_QWEN, B=64, H=2048):
    rng = np.random.default_rng(2)
    logits = rng.normal(0.0, 2.5, (B, V)).astype(np.float32)
    for r in range(B):
        peaks = rng.choice(V, 8, replace=False)
        logits[r, peaks] += np.float32(8.0)
    # One prompt token, then H generated tokens that presence and frequency
    # count (a penalty history always holds a prompt, Sampling.cpp:56-57).
    hist = rng.integers(0, V, (B, H + 1), dtype=np.int64).astype(np.uint32)
    uniforms = np.array([splitmix_uniform(row_seed(2, r), 0) for r in range(B)],
                        dtype=np.float32)
    return dict(V=V, logits=logits, histories=list(hist), generated=[H] * B,
                uniforms=uniforms,
                policy=dict(temperature=0.7, top_k=50, top_p=0.9,
                            presence=0.5, frequency=0.3),
                mark_prompt=False)


def grammar_masks(rng, B, V, fraction=0.02, singles=20):
    allowed = np.zeros((B, V), dtype=bool)
    target = int(fraction * V)
    for r in range(B):
        row = allowed[r]
        while row.sum() < target:
            start = rng.integers(0, V)
            length = rng.integers(1, 41)
            row[start:start + length] = True
        row[rng.integers(0, V, singles)] = True
    return allowed


def config3(V=V_QWEN, B=32):
    rng = np.random.default_rng(3)
    logits = to_bf16_bits(rng.normal(0.0, 2.0, (B, V)).astype(np.float32))
    allowed = grammar_masks(rng, B, V)
    uniforms = np.array([splitmix_uniform(row_seed(3, r), 0) for r in range(B)],
                        dtype=np.float32)
    return dict(V=V, logits_bf16=logits, allowed=allowed,
                masks=mask_words(allowed), uniforms=uniforms)


def random_tree(rng, rows=16, max_depth=5):
    """Parents in DFS preorder with U{1..3} children per expanded row."""
    while True:
        parent, depth = [NO_TOKEN], [0]

        def expand(r):
            if depth[r] >= max_depth:
                return
            for _ in range(int(rng.integers(1, 4))):
                if len(parent) >= rows:
                    return
                c = len(parent)
                parent.append(r)
                depth.append(depth[r] + 1)
                expand(c)

        expand(0)
        if len(parent) == rows:
            parent[0] = 0
            return parent


def chain_length(parent):
    """Rows 0..n-1 with parent[r+1] == r: the draft's first-child chain."""
    n = 1
    while n < len(parent) and parent[n] == n - 1:
        n += 1
    return n


def config4(V=V_QWEN, requests=16, rows=16, with_q=True):
    rng = np.random.default_rng(4)
    trees, tokens = [], []
    for _ in range(requests):
        parent = random_tree(rng, rows)
        trees.append(parent)
        tokens.append(rng.integers(0, V, rows, dtype=np.int64).astype(np.uint32))
    logits = rng.normal(0.0, 2.0, (requests * rows, V)).astype(np.float32)
    q = None
    if with_q:
        z = (logits - logits.mean(axis=1, keepdims=True)) / logits.std(axis=1, keepdims=True)
        e = rng.normal(0.0, 1.0, logits.shape).astype(np.float32)
        s = (0.8 * z + 0.6 * e).astype(np.float64)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        q = (p / p.sum(axis=1, keepdims=True)).astype(np.float32)
    uniforms = np.zeros((requests, 40), dtype=np.float32)
    for r in range(requests):
        c = 0
        for slot in range(1, 40):
            uniforms[r, slot] = splitmix_uniform(row_seed(4, r), c)
            c += 1
    return dict(V=V, trees=trees, tokens=tokens, logits=logits, q=q,
                uniforms=uniforms)


def config5(V=V_LARGE, B=256, H=8192):
    rng = np.random.default_rng(5)
    z = rng.normal(0.0, 1.0, (B, V)).astype(np.float32)
    t = (rng.normal(0.0, 1.0, (B, V)) /
         np.sqrt(rng.chisquare(3, (B, V)) / 3.0)).astype(np.float32)
    logits = to_bf16_bits(3.0 * z + t)
    hist = rng.integers(0, V, (B, H), dtype=np.int64).astype(np.uint32)
    uniforms = np.array([splitmix_uniform(row_seed(5, r), 0) for r in range(B)],
                        dtype=np.float32)
    return dict(V=V, logits_bf16=logits, histories=list(hist),
                generated=[H // 2] * B, uniforms=uniforms,
                policy=dict(temperature=0.8, top_k=1000, top_p=0.95, min_p=0.05,
                            repetition=1.1, presence=0.5, frequency=0.3),
                mark_prompt=True)


def config_draft(V=V_QWEN, lanes=4, seed=6):
    """The draft selector's step (DraftSelector.cpp:38-92) at the
    reference's widest batch (4 lanes): 8 fp32 query rows per lane of
    N(0, 2^2) draft logits (rows 1..7 are the proposal positions) with a few
    +6 peaks, bf16 selector hidden rows N(0, 1) and bf16 codebooks
    N(0, 0.2^2) of rank 256; lanes alternate greedy and sampled (T 0.8)."""
    rng = np.random.default_rng(seed)
    logits = rng.normal(0.0, 2.0, (lanes * 8, V)).astype(np.float32)
    peaks = rng.integers(0, V, (lanes * 8, 8))
    for r in range(lanes * 8):
        logits[r, peaks[r]] += 6.0
    hidden = to_bf16_bits(rng.normal(0.0, 1.0, (lanes * 8, 256)).astype(np.float32))
    pred = to_bf16_bits(rng.normal(0.0, 0.2, (V, 256)).astype(np.float32))
    succ = to_bf16_bits(rng.normal(0.0, 0.2, (V, 256)).astype(np.float32))
    anchors = rng.integers(0, V, lanes).astype(np.uint32)
    temperatures = [0.0 if l % 2 == 0 else 0.8 for l in range(lanes)]
    uniforms = rng.random((lanes, 40)).astype(np.float32)
    return dict(V=V, lanes=lanes, logits=logits, hidden=hidden, pred=pred, succ=succ,
                anchors=anchors, temperatures=temperatures, uniforms=uniforms)


def config_verify(V=V_LARGE, lanes=4, rows=16, H=2048):
    """The penalized chain-verify step (see the module docstring): host
    arrays in the row-indexed form of jf_sample_args (per-row draft token,
    candidate row and extra-token offset) and the acceptance inputs."""
    rng = np.random.default_rng(8)
    B = lanes * rows
    logits = rng.normal(0.0, 2.5, (B, V)).astype(np.float32)
    for g in range(B):
        logits[g, rng.choice(V, 8, replace=False)] += np.float32(8.0)
    # inputs[l * rows + i]: the lane's input i (0 the anchor, 1..15 proposals).
    inputs = rng.integers(0, V, B, dtype=np.int64).astype(np.uint32)
    for l in range(lanes):
        for r in range(rows - 1):
            logits[l * rows + r, inputs[l * rows + r + 1]] += np.float32(14.0)
    # Per row g = l * rows + r: its draft token inputs[g + 1] (rows 0..14),
    # its 16 candidates at row l * (rows - 1) + r of the lanes' candidate
    # array (the layout chain acceptance reads), its extra penalty tokens
    # inputs[l * rows + 1 ..][:r].
    P = rows - 1
    draft_index = np.full(B, NO_TOKEN, np.uint32)
    cand_index = np.zeros(B, np.uint32)
    extra_offsets = np.zeros(B, np.uint64)
    extra_counts = np.zeros(B, np.uint32)
    for l in range(lanes):
        for r in range(rows):
            g = l * rows + r
            if r < P:
                draft_index[g] = g + 1
                cand_index[g] = l * P + r
            extra_offsets[g] = l * rows + 1
            extra_counts[g] = r
    cand = rng.integers(0, V, (lanes * P, 16), dtype=np.int64).astype(np.uint32)
    for l in range(lanes):
        cand[l * P:(l + 1) * P, 0] = inputs[l * rows + 1:(l + 1) * rows]
    # The draft put about 0.6 on its proposal, the rest on the other 15.
    cprob = np.empty((lanes * P, 16), np.float32)
    cprob[:, 0] = np.float32(0.6)
    cprob[:, 1:] = (0.4 * rng.dirichlet(np.ones(15) * 0.5, lanes * P)).astype(np.float32)
    hist = rng.integers(0, V, (lanes, H), dtype=np.int64).astype(np.uint32)
    uniforms = np.zeros((lanes, 40), np.float32)
    for l in range(lanes):
        for slot in range(1, 40):
            uniforms[l, slot] = splitmix_uniform(row_seed(8, l), slot - 1)
    uniform_index = np.array([l * 40 + 15 for l in range(lanes) for _ in range(rows)],
                             np.uint32)
    return dict(V=V, lanes=lanes, rows=rows, logits=logits, inputs=inputs,
                draft_index=draft_index, cand_index=cand_index, cand_ids=cand,
                cand_probs=cprob,
                extra_offsets=extra_offsets, extra_counts=extra_counts,
                histories=list(hist), generated=[H // 2] * lanes, uniforms=uniforms,
                uniform_index=uniform_index,
                policy=dict(temperature=0.7, top_k=50, top_p=0.9, repetition=1.1,
                            presence=0.5, frequency=0.3),
                mark_prompt=True)
