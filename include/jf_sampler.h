/*
 * jf_sampler.h — C ABI of the MI355X (gfx950) logits->token path.
 *
 * The entry points replace the reference's target token policy operator
 * justfit::ops::Sampling (source/runtime/ops/Sampling.hpp:114-199) and the
 * tree acceptance dispatch Runtime::encodeTreeAcceptance
 * (source/runtime/model/Runtime.cpp:1284-1306, kernel
 * source/runtime/metal/kernels/decode/tree.metal:20-84). Every device pointer
 * is a plain HIP device address; `stream` is a hipStream_t (NULL = the null
 * stream). Calls are asynchronous on that stream unless stated otherwise.
 *
 * Errors: every function returns JF_OK (0) or a JF_ERR_* code and leaves a
 * thread-local message for jf_last_error(). Bad arguments are rejected before
 * anything is enqueued, as the reference throws std::invalid_argument before
 * it encodes (Sampling.cpp:139-142, 283-295; BufferExtent.hpp:24-28). A row
 * whose logits leave nothing to select yields JF_NO_TOKEN in-band, the
 * reference's non-finite-row sentinel (Runtime.cpp:1410-1421).
 */
#ifndef JF_SAMPLER_H
#define JF_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JF_OK 0
#define JF_ERR_INVALID_ARGUMENT 1 /* std::invalid_argument in the reference */
#define JF_ERR_LOGIC 2            /* std::logic_error in the reference */
#define JF_ERR_DEVICE 3           /* a HIP runtime call failed, or a device-side
                                     bounded wait expired (jf_sampler_status) */
#define JF_ERR_NO_MEMORY 4

#define JF_NO_TOKEN 0xffffffffu

/* Uniform slots of one lane's cycle (metal/abi/Sampling.h:19-29). */
#define JF_UNIFORM_INITIAL 0u
#define JF_UNIFORM_PROPOSALS 1u
#define JF_UNIFORM_ACCEPTANCE 8u
#define JF_UNIFORM_CORRECTION 15u
#define JF_UNIFORM_TREE_DRAWS 24u
#define JF_SAMPLING_UNIFORMS 40u
/* Draft candidates per proposal position (ExecutionGeometry.h:47). */
#define JF_DRAFT_CANDIDATES 16u
/* Penalty word layout (metal/abi/Sampling.h:111-112). */
#define JF_PENALTY_PROMPT_BIT 0x80000000u
#define JF_PENALTY_COUNT_MASK 0x7fffffffu
/* Tree geometry (metal/abi/TreeVerify.h:19-20). */
#define JF_TREE_MAXIMUM_ROWS 16u
#define JF_TREE_MAXIMUM_DEPTH 8u

#define JF_DTYPE_F32 0u
#define JF_DTYPE_BF16 1u

/* jf_policy.flags */
#define JF_POLICY_CONSTRAINED 1u  /* SamplingPolicy::constrained */
#define JF_POLICY_EXCLUDE_STOP 2u /* SamplingPolicy::excludesStopTokens */

/* One row's target policy: ops::SamplingPolicy + SamplingPenalties
 * (Sampling.hpp:19-50). temperature 0 selects greedily; top_k 0 or past the
 * vocabulary disables top-k (Sampling.cpp:23-26). */
typedef struct jf_policy {
  uint32_t top_k;
  float temperature;
  float top_p;
  float min_p;
  float repetition;
  float presence;
  float frequency;
  uint32_t flags;
} jf_policy;

typedef struct jf_sampler jf_sampler;
typedef struct jf_penalty_table jf_penalty_table;

/* The message of the calling thread's last failed call. */
const char *jf_last_error(void);

/* SamplingParameters::validationError (model/Model.hpp:77-95): JF_OK or
 * JF_ERR_INVALID_ARGUMENT with the reference's message. */
int jf_policy_validate(const jf_policy *policy);

/* ops::Sampling::Sampling(vocabulary) (Sampling.cpp:82-86), plus the device
 * scratch the reference sizes with Sampling::workspace(rows)
 * (Sampling.cpp:37-48), owned here for up to max_rows rows per call
 * (1 .. 4194304). Creates on the current HIP device; synchronous. */
int jf_sampler_create(uint32_t vocabulary, uint32_t max_rows,
                      jf_sampler **out);
int jf_sampler_destroy(jf_sampler *sampler);
/* Bytes of device scratch the sampler holds (Sampling::workspace role):
 * what jf_sampler_create allocates, plus the weights a call with drafted
 * fp32 rows and no cut had the select pass store for their residual pass
 * (4 bytes a token of those rows' chunks, allocated by the first such call
 * and grown with the rows, until jf_sampler_destroy). */
uint64_t jf_sampler_workspace_bytes(const jf_sampler *sampler);

/* No counterpart in the reference (whose last-arriving group never waits,
 * split_reduce.h:14-45). In an all-greedy jf_sample call, and for rows with
 * no cut drawn in the select launch or in the residual launch of drafted
 * rows, each row's finishing block waits, word by word, for the row's other
 * blocks' results; that wait is bounded, and the sampler holds a
 * host-mapped status word that
 * a finishing block sets if its bound is ever reached. jf_sampler_status
 * reports that as JF_ERR_DEVICE, once (jf_sample does the same before it
 * enqueues anything), and enqueues on `stream` the clearing of the words
 * such a call left. Reading the word needs no device synchronization; it
 * covers the calls whose kernels have run by then. */
int jf_sampler_status(jf_sampler *sampler, void *stream);
/* No counterpart in the reference: the bound of that wait, in reads of one
 * result word (default 2^20, about a second). It exists so that a test can
 * drive the expiry path from the host: with 0, the finishing block of every
 * such row gives up at once (it reads no other block's result) and every
 * kernel still exits normally. */
int jf_sampler_set_wait_bound(jf_sampler *sampler, uint32_t reads);

/* ---- penalties -------------------------------------------------------- */

/* Host helpers with the reference's exact semantics and errors:
 * Sampling::rebuildPenaltyWords (Sampling.cpp:50-71) and
 * Sampling::countPenaltyTokens (Sampling.cpp:75-80) over dense host words. */
int jf_penalty_words_rebuild(uint32_t *words, uint32_t vocabulary,
                             const uint32_t *history, uint64_t history_len,
                             uint64_t generated_tokens, int has_pending,
                             uint32_t pending_token, int mark_prompt);
int jf_penalty_words_count(uint32_t *words, uint32_t vocabulary,
                           const uint32_t *selected, uint64_t count);

/* The device penalty table: the reference's PenaltyTable (Sampling.hpp:55-58,
 * one dense uint32 word per vocabulary token per state lane) stored sparsely,
 * as each row's nonzero words sorted by token. Rows hold at most max_entries
 * distinct tokens. */
int jf_penalty_table_create(uint32_t vocabulary, uint32_t rows,
                            uint32_t max_entries, jf_penalty_table **out);
int jf_penalty_table_destroy(jf_penalty_table *table);
/* rebuildPenaltyWords into table row `row` from a host history (same
 * arguments, same errors); uploads on `stream`. */
int jf_penalty_table_rebuild(jf_penalty_table *table, uint32_t row,
                             const uint32_t *history, uint64_t history_len,
                             uint64_t generated_tokens, int has_pending,
                             uint32_t pending_token, int mark_prompt,
                             void *stream);
/* countPenaltyTokens (Sampling.cpp:75-80) of `count` host tokens into table
 * row `row`, in order; Runtime.cpp:1397-1406 (commitSelected) is the call
 * site it serves. The table is updated in place on `stream` by one kernel
 * launch: up to 64 tokens' updates travel as kernel arguments; a call with
 * more puts them in host-mapped pinned memory that the kernel reads (four
 * such buffers a table, each reused once the launch that read it has
 * completed: the only wait on earlier work). Nothing of the row is
 * uploaded. Calls on one table must be ordered (one stream, or streams
 * ordered by the caller). Only calls of up to 64 tokens may be captured
 * into a HIP graph: a longer call's kernel reads its updates at run time
 * from a buffer that later calls reuse. (Once in a table's life, when a row first needs more
 * than 256 of a chunk's fixed slots and 512 suffice, a rebuild or count
 * widens them to 512 and uploads every row's slots.) All-or-nothing: a
 * token outside the vocabulary, or new tokens beyond the row's
 * max_entries, fail before the row changes. */
int jf_penalty_table_count(jf_penalty_table *table, uint32_t row,
                           const uint32_t *selected, uint64_t count,
                           void *stream);
/* The same for one step's commits of every lane at once: pair i counts
 * token selected[i] into row rows[i] (rows may repeat; each row's tokens
 * apply in order). One launch per call. */
int jf_penalty_table_count_rows(jf_penalty_table *table, const uint32_t *rows,
                                const uint32_t *selected, uint64_t count,
                                void *stream);

/* ---- uniforms --------------------------------------------------------- */

/* Runtime::nextUniform (Runtime.cpp:1098-1105): SplitMix64 of
 * seed + (++counter) * 0x9e3779b97f4a7c15, top 24 bits scaled by 2^-24. */
float jf_next_uniform(uint64_t seed, uint64_t *counter);
/* Runtime::stageSamplingCycle (Runtime.cpp:1107-1114) into 40 host floats. */
void jf_stage_sampling_cycle(uint64_t seed, uint64_t *counter,
                             uint32_t verify_rows, int tree_cycle,
                             float *uniforms40);

/* ---- selection -------------------------------------------------------- */

/* One selection over `rows` rows: what Sampling::addInitial and
 * Sampling::addVerify encode (Sampling.cpp:134-172, 244-276) — penalties,
 * then each greedy row's argmax or each sampled row's min-p/top-k/top-p draw
 * — generalized from <= 4 lanes x 8/16 rows to `rows` independent rows with
 * explicit strides. Row r reads:
 *   logits  + r * logits_stride   (elements of dtype; 16-byte aligned rows)
 *   masks   + r * mask_stride     (uint32 words; constrained rows only)
 *   uniforms[uniform_index ? uniform_index[r]
 *            : uniform_offset + r * uniform_stride]   (sampled rows; a
 *   stride of 0 gives every row the same uniform, the reference's
 *   correction slot; stride 1 with offset 24 its per-row tree draws)
 *   penalty table row penalty_rows[r] and extra_tokens + r * extra_stride
 *   (extra_counts[r] tokens each counted once more: the draft tokens a
 *   verify row's context adds, Sampling.cpp:118-131, sampling.metal:978-993)
 *   draft_tokens[r] for r < drafted_rows: JF_NO_TOKEN, or the draft token
 *   the row's draw corrects (TargetSamplingParams::drafted_rows: a drafted
 *   verify row); rows from drafted_rows on are not drafted; the draft
 *   distribution is dense
 *   (draft_q + r * draft_q_stride) when draft_q is set, else the sparse
 *   candidates draft_cand_ids/probs + r * JF_DRAFT_CANDIDATES.
 * Writes out_tokens[r] and, when set, out_draft_probs[r] (the target's
 * probability of the row's draft token, TargetVocabularyRow::draft_probability)
 * and the kept distribution (out_kept_counts[r]; ids ascending and their
 * probabilities in out_kept_ids/out_kept_probs + r * kept_capacity).
 * The logits are read-only: the reference rewrites penalized logits in place,
 * this build applies penalties on the fly. */
typedef struct jf_sample_args {
  uint32_t rows;
  uint32_t dtype;
  const void *logits;
  uint64_t logits_stride;
  const uint32_t *masks;
  uint64_t mask_stride;
  const jf_policy *policies;       /* host, rows entries */
  uint32_t stop_token_0;
  uint32_t stop_token_1;
  const jf_penalty_table *penalties;
  const uint32_t *penalty_rows;    /* host, rows entries, or NULL */
  const uint32_t *extra_tokens;    /* device */
  const uint32_t *extra_counts;    /* host, rows entries (<= 16), or NULL */
  uint64_t extra_stride;
  const float *uniforms;           /* device */
  const uint32_t *uniform_index;   /* device, or NULL */
  uint64_t uniform_offset;
  uint64_t uniform_stride;
  const uint32_t *draft_tokens;    /* device, or NULL */
  uint32_t drafted_rows;
  const uint32_t *draft_cand_ids;  /* device */
  const float *draft_cand_probs;   /* device */
  const float *draft_q;            /* device, or NULL */
  uint64_t draft_q_stride;
  uint32_t *out_tokens;            /* device */
  float *out_draft_probs;          /* device, or NULL */
  uint32_t *out_kept_counts;       /* device, or NULL */
  uint32_t *out_kept_ids;          /* device */
  float *out_kept_probs;           /* device */
  uint32_t kept_capacity;
  /* Optional, with no counterpart in the reference: two hipEvent_t that the
   * single-pass selection kernel's launch records at its own start and end
   * (hipExtLaunchKernelGGL), so that a caller can time that kernel alone.
   * Both NULL records nothing. */
  void *select_start_event;
  void *select_done_event;
  /* Optional per-row addressing (host arrays of `rows` entries, or NULL for
   * the linear forms above), so that one call covers every lane of a verify
   * batch as the reference's one dispatch set does (Sampling.cpp:149-172;
   * row addressing sampling.metal:52-70, 912-913):
   *   mask_rows[r]          row r's mask is masks + mask_rows[r] * mask_stride
   *   draft_token_index[r]  row r's draft token is draft_tokens[index], or
   *                         JF_NO_TOKEN for an undrafted row (replaces
   *                         drafted_rows)
   *   draft_cand_index[r]   its draft distribution: draft_cand_ids/probs +
   *                         index * JF_DRAFT_CANDIDATES, or dense row index
   *   extra_offsets[r]      its extra tokens start at extra_tokens + offset
   *                         (replaces r * extra_stride) */
  const uint32_t *mask_rows;
  const uint32_t *draft_token_index;
  const uint32_t *draft_cand_index;
  const uint64_t *extra_offsets;
} jf_sample_args;

/* Selection of every row of `args` on `stream`, asynchronous.
 *
 * Stream contract: one sampler's scratch (row parameters, chunk summaries,
 * candidate lists, counters, packed bests) is shared by every call on it, so
 * calls on one sampler must be ordered: issued on one stream, or on streams
 * the caller orders (events). Two unordered calls on one sampler race. This
 * is the reference's own model: one engine thread records every selection
 * into one command graph (Sampling.hpp:114-199; Runtime.cpp:2290-2295).
 * Separate samplers are independent.
 *
 * In an all-greedy call each row's finishing block (its last chunk, or its
 * last block to arrive) waits for the row's other blocks' results. Blocks
 * are dispatched in the order of their index, chunk fastest, so the blocks
 * a finisher waits for were dispatched before it, and they wait on nothing:
 * every wait ends. The wait is still bounded; should the bound ever be
 * reached, the row gets JF_NO_TOKEN and the sampler's status word is set,
 * which the next jf_sample (or jf_sampler_status) reports as JF_ERR_DEVICE
 * before enqueuing anything else. */
int jf_sample(jf_sampler *sampler, const jf_sample_args *args, void *stream);

/* jf_sample without a sampler object and without any allocation. It has no
 * counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The scratch that jf_sampler_create would
 * allocate is instead one file-scope device array of 21,065,984 bytes, held
 * by every GPU the library runs on until the process ends. Limits: 1..64
 * rows and a vocabulary of 1..262,144 tokens; larger calls return
 * JF_ERR_INVALID_ARGUMENT. The caller still passes inputs and outputs (and
 * any penalty table, created beforehand). Same arguments, results and errors
 * as jf_sample otherwise. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (on different streams) race; calls in one
 * stream's order do not. It has no status word: should a finisher's
 * bounded wait ever expire (an all-greedy row's, or a row with no cut drawn
 * in the select or residual launch), that row's output is JF_NO_TOKEN
 * (in-band, as the reference reports numeric failures) and nothing else
 * reports it. */
int jf_sample_static(uint32_t vocabulary, const jf_sample_args *args, void *stream);

/* ---- acceptance ------------------------------------------------------- */

/* Sampling::addAcceptance (Sampling.cpp:278-328) -> decode_accept_dflash
 * (sampling.metal:1528-1558) over `lanes` lanes of verify_rows (8 or 16)
 * rows. Per lane l: proposed_tokens + l*(verify_rows-1), candidates and
 * proposal_probs + l*(verify_rows-1)*16, target_draft_probs +
 * l*verify_rows (the selection's out_draft_probs), uniforms + l*40,
 * target_tokens + l*verify_rows (in: the selection's tokens; out: the
 * accepted chain). maximum_retained and policies are host arrays. */
typedef struct jf_accept_chain_args {
  uint32_t lanes;
  uint32_t verify_rows;
  const uint32_t *proposed_tokens;
  const uint32_t *candidates;
  const float *proposal_probs;
  const float *target_draft_probs;
  const float *uniforms;
  uint32_t *target_tokens;
  uint32_t *retained_counts;
  uint32_t *accepted_counts;
  const uint32_t *maximum_retained; /* host */
  const jf_policy *policies;        /* host */
  uint32_t stop_token_0;
  uint32_t stop_token_1;
} jf_accept_chain_args;

int jf_accept_chain(jf_sampler *sampler, const jf_accept_chain_args *args,
                    void *stream);

/* One lane's draft tree: the fields of JustFitTreeLane that acceptance reads
 * (TreeVerify.h:22-31) and the sampled chain of JustFitTreeAcceptParams
 * (TreeVerify.h:40-52). Rows in DFS preorder, parent[r] < r, row 0 the
 * anchor; rows 0 .. chain_rows-1 are the draft's sampled chain and chain_q[r]
 * is the draft probability of row r+1's token. */
typedef struct jf_tree_lane {
  uint32_t rows;
  uint32_t chain_rows;
  uint32_t parent[JF_TREE_MAXIMUM_ROWS];
  uint32_t token[JF_TREE_MAXIMUM_ROWS];
  float chain_q[JF_TREE_MAXIMUM_DEPTH];
} jf_tree_lane;

/* verify_tree_accept (tree.metal:20-84) over `lanes` lanes. Per lane l:
 * trees[l] (host), target_tokens + l*rows_per_lane (in: each row's selected
 * token; out: the accepted path's tokens then the bonus token),
 * target_draft_probs + l*rows_per_lane, uniforms + l*40, path_rows + l*8. */
typedef struct jf_accept_tree_args {
  uint32_t lanes;
  uint32_t rows_per_lane;
  const jf_tree_lane *trees;        /* host */
  const float *target_draft_probs;
  const float *uniforms;
  uint32_t *target_tokens;
  uint32_t *retained_counts;
  uint32_t *accepted_counts;
  uint32_t *path_rows;
  const uint32_t *maximum_retained; /* host */
  const jf_policy *policies;        /* host */
  uint32_t stop_token_0;
  uint32_t stop_token_1;
} jf_accept_tree_args;

int jf_accept_tree(jf_sampler *sampler, const jf_accept_tree_args *args,
                   void *stream);

/* No single counterpart in the reference, whose engine records the
 * selection (Sampling::addInitial/addVerify) and verify_tree_accept into one
 * command buffer (Runtime.cpp:1284-1306): jf_sample(sample) then
 * jf_accept_tree(accept) on `stream`, with the same results, as one launch
 * when it can: every lane greedy, the lanes' rows the selection's rows in
 * order (lanes x rows_per_lane == rows, accept->target_tokens ==
 * sample->out_tokens, at most 16 lanes), and the selection a uniform
 * all-greedy launch that each row's last chunk block finishes. Then the
 * finisher of each lane's last row gathers the lane's tokens and walks the
 * tree. Otherwise the two calls run one after the other. A bounded wait
 * that gives up leaves the lane's rows JF_NO_TOKEN and is reported as for
 * jf_sample. */
int jf_sample_accept_tree(jf_sampler *sampler, const jf_sample_args *sample,
                          const jf_accept_tree_args *accept, void *stream);

/* ---- draft selector ---------------------------------------------------- */

/* The DFlash draft's proposal policy: ops::DraftSelector
 * (source/runtime/ops/DraftSelector.hpp:41-60, DraftSelector.cpp:22-92),
 * kernels draft_select_top16_sharded / draft_select_edges /
 * draft_select_dflash (sampling.metal:995-1359). Lane geometry as in
 * ExecutionGeometry.h: 8 query rows, 7 proposal positions, 16 candidates per
 * position, selector rank 256. */
#define JF_DRAFT_QUERY_ROWS 8u
#define JF_DRAFT_POSITIONS 7u
#define JF_DRAFT_SELECTOR_RANK 256u

typedef struct jf_draft_selector jf_draft_selector;

/* DraftSelector::DraftSelector(vocabulary) (DraftSelector.cpp:22-25), plus
 * the scratch DraftSelector::workspace sizes (DraftSelector.cpp:27-36),
 * owned here for up to max_lanes lanes per call. Creates on the current HIP
 * device; synchronous. */
int jf_draft_selector_create(uint32_t vocabulary, uint32_t max_lanes,
                             jf_draft_selector **out);
int jf_draft_selector_destroy(jf_draft_selector *selector);

/* DraftSelector::add (DraftSelector.cpp:38-92) over `lanes` lanes. Lane l
 * reads its query rows logits + (l*8 + r) * logits_stride (fp32; rows 1..7
 * are proposal positions 0..6) and selector_hidden + (l*8 + r) * 256 (bf16
 * bits), the bf16 codebooks [vocabulary][256] (16-byte aligned), anchors[l]
 * and policies[l] (host; temperature 0 walks greedily, otherwise the lane
 * draws with uniforms + l*40 + JF_UNIFORM_PROPOSALS + position). Writes, per
 * proposal row s = l*7 + position: candidates + s*16 and unary + s*16 (the
 * row's top 16 in (logit desc, id asc) order and their logits; slots past
 * the row's non-NaN tokens hold JF_NO_TOKEN and -inf), proposed_tokens[s],
 * and for a sampling lane proposal_probs + s*16 (the walk's candidate
 * probabilities). Each edge score is the fp32 sum over the rank, in
 * ascending order, of (predecessor codebook x hidden) x successor codebook;
 * ids are clamped into the codebooks as the reference does. Optional
 * select_start_event/select_done_event (hipEvent_t, with no counterpart in
 * the reference) bracket the top-16 kernel. */
typedef struct jf_draft_select_args {
  uint32_t lanes;
  const float *logits;                   /* device */
  uint64_t logits_stride;                /* elements, >= vocabulary */
  const uint16_t *selector_hidden;       /* device */
  const uint16_t *predecessor_codebook;  /* device */
  const uint16_t *successor_codebook;    /* device */
  const uint32_t *anchors;               /* host, lanes entries */
  const jf_policy *policies;             /* host, lanes entries */
  const float *uniforms;                 /* device; needed when a lane samples */
  uint32_t *candidates;                  /* device */
  float *unary;                          /* device */
  uint32_t *proposed_tokens;             /* device */
  float *proposal_probs;                 /* device; needed when a lane samples */
  void *select_start_event;
  void *select_done_event;
  /* Optional (device, [lanes][7][16][16], or NULL): the edge tables, entry
   * (p, i, j) the score from predecessor i to candidate j at position p, for
   * jf_build_draft_tree. Position 0 has only predecessor 0 (the anchor); its
   * other rows are left unwritten. */
  float *edge_tables;
} jf_draft_select_args;

int jf_draft_select(jf_draft_selector *selector,
                    const jf_draft_select_args *args, void *stream);

/* ---- draft tree builder ------------------------------------------------- */

/* One lane's draft tree in its verify rows: JustFitTreeLane
 * (metal/abi/TreeVerify.h:14-32). Rows are in DFS preorder: row 0 is the
 * anchor (depth 0) and every row's parent row is smaller than the row. A copy
 * is one root-to-leaf path; path[c][d] is its row at depth d. Every row
 * belongs to the first copy, in DFS order, whose path holds it. */
typedef struct jf_draft_tree {
  uint32_t rows;
  uint32_t copies;
  uint32_t parent[JF_TREE_MAXIMUM_ROWS];
  uint32_t depth[JF_TREE_MAXIMUM_ROWS];
  uint32_t copy[JF_TREE_MAXIMUM_ROWS];
  uint32_t token[JF_TREE_MAXIMUM_ROWS];
  uint32_t path_length[JF_TREE_MAXIMUM_ROWS];
  uint32_t path[JF_TREE_MAXIMUM_ROWS][JF_TREE_MAXIMUM_DEPTH];
} jf_draft_tree;

/* buildDraftTree (source/runtime/model/Runtime.cpp:58-174), host only and
 * synchronous: one lane's tree of at most `rows` (1..16) rows from the draft
 * selector's candidates [7][16] and unary scores [7][16] (jf_draft_select's
 * outputs) and its edge tables [7][16][16] (entry (p, i, j): predecessor i to
 * candidate j at position p; position 0 reads predecessor 0, the anchor).
 * Nodes are taken best first by path log-probability (double), children of a
 * node scored by a log-softmax over its 16 candidates. chain_picks (7
 * candidate indices, or NULL) forces a sampled lane's chain as the leftmost
 * path. expected / chain_expected (optional) receive the sum of the tree's
 * node probabilities and that of the selector's own greedy chain. */
int jf_build_draft_tree(const uint32_t *candidates, const float *unary,
                        const float *edges, uint32_t anchor, uint32_t rows,
                        const uint32_t *chain_picks, jf_draft_tree *out,
                        double *expected, double *chain_expected);

/* ---- mask wire format --------------------------------------------------- */

/* The frames between the engine's grammar and the runtime
 * (source/runtime/engine/Protocol.hpp:22-25, 34-50, 185-203, 263-278): a
 * 16-byte header ("SPLH", u16 protocol version 9, u16 frame type, u64
 * payload bytes), then the payload; every integer little-endian. */
#define JF_FRAME_MASK_RESPONSE 0x0003u
#define JF_FRAME_MASK_REQUEST 0x0103u
#define JF_FRAME_MASK_TREE_REQUEST 0x0109u

/* encodeMaskRequest (Protocol.cpp:616-632) with validateMaskRequest
 * (Protocol.cpp:469-500) at the default ProtocolLimits: payload u64
 * request_id, u64 mask_request_id, u32 words_per_mask, u32 count, count u32
 * simulation tokens, and for a tree (parents != NULL, MaskTreeRequest) count
 * u32 parents (parents[0] == 0, parents[r] < r). `written` receives the frame
 * bytes. */
int jf_mask_request_encode(uint64_t request_id, uint64_t mask_request_id,
                           uint32_t words_per_mask, const uint32_t *tokens,
                           uint32_t count, const uint32_t *parents,
                           uint8_t *out, uint64_t capacity, uint64_t *written);

/* decodeMaskResponse (Protocol.cpp:793-820) with validateMaskResponse
 * (402-414) of one whole MaskResponse frame: payload u64 request_id, u64
 * mask_request_id, u32 count, count u32 mask words (into words, capacity
 * words). */
int jf_mask_response_decode(const uint8_t *frame, uint64_t bytes,
                            uint64_t *request_id, uint64_t *mask_request_id,
                            uint32_t *words, uint32_t capacity, uint32_t *count);

/* Runtime::provideMask's checks (Runtime.cpp:3466-3481) on `rows` mask rows
 * of mask_words words: every row admits a token, and for a verify mask
 * (pending_token != JF_NO_TOKEN) row 0 admits the pending anchor. The rows
 * are then the `masks` of jf_sample (mask_stride = mask_words). */
int jf_mask_rows_check(const uint32_t *words, uint32_t rows,
                       uint32_t mask_words, uint32_t pending_token);

/* The row rules of the engine's masks (rust/frontend/src/grammar.rs:222-270),
 * in place on count + 1 rows of mask_words words. Chain: rows 0..valid hold
 * the masks after 0..valid accepted simulation tokens; rows past valid
 * repeat row valid. Tree: row 0 is the state before the anchor and row r + 1
 * the state after token row r's path; a token row whose own token is
 * refused[r], or whose parent row is itself refused, takes the mask of its
 * parent's row (row 0 for the anchor). */
int jf_mask_chain_fill(uint32_t *words, uint32_t count, uint32_t valid,
                       uint32_t mask_words);
int jf_mask_tree_fill(uint32_t *words, uint32_t count, const uint32_t *parents,
                      const uint8_t *refused, uint32_t mask_words);

/* ---- tree gather -------------------------------------------------------- */

/* verify_tree_gather (tree.metal:86-107), which Runtime::encodeTreeGathers
 * (Runtime.cpp:1311-1341) dispatches once per tensor family: in place, each
 * lane's accepted path rows move to rows 0 .. retained - 1. The layout fields
 * are JustFitTreeGatherParams (metal/abi/TreeVerify.h:54-69), in 16-bit
 * units: element (row, column) of lane b and layer y sits at
 *   y*layer_stride + b*lane_stride + row*row_stride
 *   + (column / inner)*outer_stride + (column % inner)*inner_stride.
 * path_rows + b*8 and retained[b] are jf_accept_tree's outputs (device).
 * With no counterpart in the reference, for the extent check and device
 * safety: data_units (elements in data) and rows (rows per lane of the
 * tensor, 1..16; a path row at or past it is skipped). Optional
 * start_event/done_event (hipEvent_t) bracket the kernel. */
typedef struct jf_tree_gather_args {
  uint16_t *data;
  uint64_t data_units;
  const uint32_t *path_rows;
  const uint32_t *retained;
  uint32_t columns;
  uint32_t inner;
  uint32_t inner_stride;
  uint32_t outer_stride;
  uint32_t row_stride;
  uint32_t lane_stride;
  uint32_t layer_stride;
  uint32_t layers;
  uint32_t lanes;
  uint32_t rows;
  void *start_event;
  void *done_event;
} jf_tree_gather_args;

int jf_tree_gather(const jf_tree_gather_args *args, void *stream);

#ifdef __cplusplus
}
#endif
#endif
