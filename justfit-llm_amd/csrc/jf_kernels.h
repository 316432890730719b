// Shared declarations of the gfx950 sampler: the device parameter records
// the host builds, the scratch records the kernels exchange, and the launch
// entry points of jf_kernels.hip.
#pragma once

#include <stdint.h>

#include "jf_host.h"

struct jf_sample_args;

namespace jf {

// Per-row target policy as the kernels read it (the reference's
// TargetSamplingParams + SamplingPenaltyParams fields of one lane,
// metal/abi/Sampling.h:40-61, 118-129), derived on the host.
struct RowParams {
  uint32_t flags;
  uint32_t top_k;             // effective: the vocabulary when disabled
  float inv_t;                // 1 / temperature
  float top_p;
  float minp_offset;          // temperature * log(min_p)
  float repetition;
  float repetition_inverse;   // min(1 / repetition, FLT_MAX)
  float presence;
  float frequency;
  uint32_t penalty_row;
  uint32_t extra_count;
  uint32_t extra_offset;      // the row's extra tokens: SampleLaunch::extra + this
  uint32_t draft_index;       // its draft token: draft_tokens[draft_index]
                              // (kNoToken: not drafted)
  uint32_t cand_index;        // its draft distribution: sparse candidates
                              // cand_ids/probs + 16 * this, dense q row this
  uint32_t mask_row;          // its constraint mask: masks + this * mask_stride
  uint32_t fast_row;          // nonzero: a launch split between the two select
                              // kernels selects this row in the fast one
};
static_assert(sizeof(RowParams) == 64, "row params are 64 bytes");

enum RowFlags : uint32_t {
  kRowSampled = 1u,
  kRowConstrained = 2u,
  kRowExcludeStop = 4u,
  kRowPenalized = 8u,
  kRowMinP = 16u,
  kRowTopP = 32u,
  kRowTopK = 64u,
  // A drafted row with no cut, penalty, mask or extra tokens: its residual
  // pass runs in residual_kernel (set by the host).
  kRowLean = 128u,
};

// One block's summary of its chunk of a row.
struct BlockHeader {
  float maximum;       // sampled: largest admitted logit (-FLT_MAX if none)
  uint32_t count;      // sampled: candidates written
  uint32_t admitted;   // sampled: 1 when the chunk admits a non-NaN token
  uint32_t overflow;   // sampled: candidates did not fit
  float best_value;    // greedy
  uint32_t best_id;    // greedy
  uint32_t floor_key;  // sampled: the row's K-th key is at least this
  uint32_t reserved;
};
static_assert(sizeof(BlockHeader) == 32, "block headers are 32 bytes");

// A row the single pass could not finish: the multi-pass stages carry it.
struct RowState {
  uint32_t stage;
  float maximum;
  uint32_t thr_key;      // min-p floor key, 0 without min-p
  uint32_t bkey;         // kept set boundary in (key desc, id asc) order
  uint32_t bid;
  uint32_t prefix;       // radix descent
  uint32_t pmask;
  uint32_t chunk;        // the chunk a locate or walk stage works in
  uint64_t remaining;    // radix descent: count or mass still to place
  uint64_t n1;           // tokens at or above the min-p floor
  uint64_t mass2;
  uint64_t nucleus;
  uint64_t mass3;
  uint64_t target;
  uint64_t within;       // target or rank inside `chunk`
  uint32_t tie_key;
  uint32_t residual;
  float draft_w;
  uint32_t drafted;
  uint64_t reserved[3];
};
static_assert(sizeof(RowState) == 128, "row states are 128 bytes");

struct StagePartial {
  uint64_t v[256];
};

// Geometry of one selection launch.
constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kBlockCandidates = 1024;
constexpr int kMergeCapacity = 2048;
constexpr int kPenaltyWordsLds = 2048;
constexpr int kMaxExtra = 16;
constexpr uint32_t kChunkF32 = 8192;
constexpr uint32_t kChunkBF16 = 8192;

struct SampleLaunch {
  const void *logits;
  uint64_t stride;
  const uint32_t *masks;
  uint64_t mask_stride;
  const RowParams *params;
  uint32_t vocabulary;
  uint32_t chunks;
  uint32_t rows;
  uint32_t stop0;
  uint32_t stop1;
  uint32_t stage;
  uint32_t aligned;       // rows start on 16-byte boundaries: vector loads
  uint32_t finish_greedy; // no merge runs: uncut_kernel finishes the greedy
                          // rows
  uint32_t row_indexed;   // drafts are addressed through RowParams'
                          // draft_index/cand_index, not the row number
  const uint2 *pen_entries;
  const uint32_t *pen_offsets;
  uint32_t pen_max_entries;
  uint32_t pen_buckets;
  const uint32_t *extra;
  uint64_t extra_stride;
  const float *uniforms;
  const uint32_t *uniform_index;
  uint64_t uniform_offset;
  uint64_t uniform_stride;
  const uint32_t *draft_tokens;
  uint32_t drafted_rows;
  const uint32_t *cand_ids;
  const float *cand_probs;
  const float *dense_q;
  uint64_t q_stride;
  BlockHeader *headers;
  uint64_t *cands;       // key | id << 32
  uint32_t *counters;
  uint64_t *bests;       // all-greedy fast launches: each block's packed best
                         // (zero between calls unless a wait gave up)
  RowState *states;
  StagePartial *partials;
  uint32_t *out_tokens;
  float *out_draft;
  uint32_t *out_kept_counts;
  uint32_t *out_kept_ids;
  float *out_kept_probs;
  uint32_t kept_cap;
  uint32_t q_aligned;     // dense q rows start on 16-byte boundaries
  uint32_t epoch;         // the call's tag of its packed greedy bests (1..4095)
  uint32_t wait_bound;    // reads of a packed best before its wait gives up
  uint32_t *status;       // set to 1 when a wait gave up (host-mapped), or NULL
  // Drafted rows with no cut (kRowLean) in an all-fast fp32 launch: the
  // select pass also stores each token's weight there as pack_yk (row r at
  // r * lean_stride, chunk-major like the logits), and residual_kernel
  // reads it instead of the logits; NULL otherwise.
  uint32_t *lean_weights;
  uint64_t lean_stride;
};

// The fast selection launch: the per-row facts every block needs before its
// first load (flags, penalty table row) travel in the kernel arguments, and
// each (table row, chunk) holds its penalty entries in a fixed run of
// `slot_count` 32-bit slots, so a block requests them together with its
// logits and waits on nothing first. Slot = offset in the chunk << 19 |
// prompt bit << 18 | count (< 2^18); an empty slot is 0 (every real entry
// has a count or the prompt bit). A uniform launch (every row the same
// policy, each reading its own penalty row, no row map, no extra tokens)
// carries no per-row facts (FastRows) at all: the kernel-argument segment
// the runtime copies for every launch then stays small.
constexpr int kKernargRows = 256;
struct FastLaunch {
  SampleLaunch a;
  const uint32_t *pen_slots;  // [table rows][chunks][slot_count]
  uint32_t slot_count;        // 256 or 512
  uint32_t row_base;          // sampler row of blockIdx.y == 0
  uint32_t fuse_greedy;       // every row greedy, no merge launch: 1, the
                              // row's last block to arrive finishes it; 2
                              // (set at launch when its rows are fewer than
                              // the blocks the GPU holds at once), the
                              // row's last chunk finishes it
  uint32_t mapped;            // blockIdx.y selects row row_of[blockIdx.y]
                              // (a launch split between the two kernels;
                              // the kernel takes it as a preloaded argument)
  uint32_t lean_bits[kKernargRows / 32];  // bit y: row blockIdx.y stores its
                                          // weights (a.lean_weights)
};
// The per-row facts of a launch that is not uniform, by blockIdx.y.
struct FastRows {
  uint32_t row_info[kKernargRows];  // RowFlags | penalty row << 8
  uint32_t row_of[kKernargRows];
  // Launches whose rows carry extra (verify) penalty tokens: the row's
  // extras are SampleLaunch::extra + (this & kExtraOffsetMask), this >> 27
  // of them (<= kMaxExtra).
  uint32_t row_extra[kKernargRows];
};
// The argument a uniform launch passes in FastRows' place.
struct NoRows {};
// The fast selection's last argument, naming what its finishing blocks do
// beyond selecting: nothing more, draw rows with no cut (UncutFinish), or
// (an AcceptTreeLaunch) run each lane's tree acceptance; StoreWeights is
// NoFinish that also stores the drafted rows' weights (a.lean_weights), a
// separate instantiation since the stores take registers.
struct NoFinish {};
struct UncutFinish {};
struct StoreWeights {};
constexpr uint32_t kExtraOffsetMask = (1u << 27) - 1u;

// Multi-pass stages, in launch order.
enum Stage : uint32_t {
  kStageDone = 0,
  kStageCount1 = 1,
  kStageTopK3 = 2,
  kStageTopK0 = 5,
  kStageTopKTie = 6,
  kStageTopKLocate = 7,
  kStageMass2 = 8,
  kStageTopP3 = 9,
  kStageTopP0 = 12,
  kStageTopPTie = 13,
  kStageTopPLocate = 14,
  kStageMass3 = 15,     // picks the draw's chunk for a row without a draft
  kStageDraw = 16,      // drafted rows: residual masses, the draw's chunk
  kStageWalk = 17,      // one block per row: the draw inside its chunk
  kStageKeptCount = 18,
  kStageKeptWrite = 19,
  kStageLast = 19,
};

// Classes of stages that share code (one stage-kernel build each).
enum StageClass : int {
  kClsCount = 0,     // kStageCount1
  kClsDigits = 1,    // radix digits of the k-th key and of the nucleus
  kClsTie = 2,       // ties at the boundary key
  kClsLocate = 3,    // the boundary token inside one chunk
  kClsMass = 4,      // kStageMass2, kStageMass3, kStageKeptCount
  kClsDraw = 5,
  kClsKeptWrite = 6,
  kClsWalk = 7,      // walk_kernel, not a stage_kernel build
  kClsNone = 8,
};
__host__ __device__ constexpr int stage_class(uint32_t stage) {
  return stage == kStageCount1 ? kClsCount
         : (stage >= kStageTopK3 && stage <= kStageTopK0) ||
                   (stage >= kStageTopP3 && stage <= kStageTopP0)
             ? kClsDigits
         : stage == kStageTopKTie || stage == kStageTopPTie       ? kClsTie
         : stage == kStageTopKLocate || stage == kStageTopPLocate ? kClsLocate
         : stage == kStageMass2 || stage == kStageMass3 || stage == kStageKeptCount
             ? kClsMass
         : stage == kStageDraw      ? kClsDraw
         : stage == kStageKeptWrite ? kClsKeptWrite
         : stage == kStageWalk      ? kClsWalk
                                    : kClsNone;
}

struct AcceptChainLane {
  uint32_t remaining;
  uint32_t sampled;
};

// Chain acceptance: up to kChainLanesPerLaunch lanes a launch, their
// records in the kernel arguments (no upload); the pointers start at the
// launch's first lane.
constexpr uint32_t kChainLanesPerLaunch = 256;
struct AcceptChainLaunch {
  uint32_t lanes;
  uint32_t verify_rows;
  const uint32_t *proposed;
  const uint32_t *candidates;
  const float *proposal_probs;
  const float *target_draft_probs;
  const float *uniforms;
  uint32_t *target_tokens;
  uint32_t *retained;
  uint32_t *accepted;
  uint32_t stop0;
  uint32_t stop1;
  AcceptChainLane lane_params[kChainLanesPerLaunch];
};

struct TreeLaneParams {
  uint32_t rows;
  uint32_t chain_rows;
  uint32_t remaining;
  uint32_t sampled;
  uint32_t parent[16];
  uint32_t token[16];
  float chain_q[8];
};

// Tree acceptance: up to kTreeLanesPerLaunch lanes a launch, their trees in
// the kernel arguments; the pointers start at the launch's first lane.
constexpr uint32_t kTreeLanesPerLaunch = 16;
struct AcceptTreeLaunch {
  uint32_t lanes;
  uint32_t rows_per_lane;
  const float *target_draft_probs;
  const float *uniforms;
  uint32_t *target_tokens;
  uint32_t *retained;
  uint32_t *accepted;
  uint32_t *path_rows;
  uint32_t stop0;
  uint32_t stop1;
  TreeLaneParams trees[kTreeLanesPerLaunch];
};

// The draft selector (jf_draft.hip): lane geometry of the reference's DFlash
// draft (ExecutionGeometry.h: 8 query rows, 7 proposal positions, 16
// candidates, selector rank 256) and the uniform slots of a lane
// (metal/abi/Sampling.h:19-29).
constexpr uint32_t kDraftQueryRows = 8;
constexpr uint32_t kDraftPositions = 7;
constexpr uint32_t kSamplingUniforms = 40;
constexpr uint32_t kUniformProposals = 1;
struct DraftLaneParams {
  uint32_t anchor;
  float temperature;
  uint32_t sampled;
  uint32_t reserved;
};
struct DraftLaunch {
  const float *logits;        // [lanes * 8][stride]
  uint64_t stride;
  uint32_t vocabulary;
  uint32_t chunks;            // 8192-token chunks per row
  uint32_t lanes;
  const uint16_t *hidden;     // bf16 [lanes * 8][256]
  const uint16_t *pred_codebook;  // bf16 [vocabulary][256]
  const uint16_t *succ_codebook;  // bf16 [vocabulary][256]
  const DraftLaneParams *lane_params;
  const float *uniforms;      // [lanes][40]
  uint32_t *candidates;       // [lanes * 7][16]
  float *unary;               // [lanes * 7][16]
  uint32_t *tokens;           // [lanes * 7]
  float *q_probs;             // [lanes * 7][16], sampled lanes
  uint64_t *part_comp;        // [lanes * 7][chunks][16]
  uint32_t *part_vbits;       // [lanes * 7][chunks][16]
  float *tables;              // [lanes][7][16][16]
  uint32_t *choices;          // [lanes * 7][16]: the walk's pick after each predecessor
  float *choice_q;            // [lanes * 7][16][16]: its probabilities, sampled lanes
  uint32_t *counters;         // [lanes * 8], zero between launches
};

// The tree gather (jf_gather.hip): JustFitTreeGatherParams (TreeVerify.h:54-69)
// in 16-bit units, plus the rows per lane of the tensor.
constexpr uint32_t kGatherDepth = 8;  // path entries per lane
struct GatherLaunch {
  uint16_t *data;
  const uint32_t *path_rows;  // [lanes][8]
  const uint32_t *retained;   // [lanes]
  uint32_t columns, inner, inner_stride, outer_stride;
  uint64_t row_stride, lane_stride, layer_stride;
  uint32_t layers, lanes, rows;
};

// The device scratch of one selection: where its kernels exchange row
// parameters, chunk summaries, candidate lists, arrival counters and packed
// greedy bests (both zero between calls), row states and stage partials. Room for max_rows rows of
// at most max_chunks 8192-token chunks.
struct SampleScratch {
  RowParams *params;        // [max_rows]
  BlockHeader *headers;     // [max_rows * max_chunks]
  uint64_t *cands;          // [max_rows * max_chunks * kBlockCandidates]
  uint32_t *counters;       // [max_rows]
  uint64_t *bests;          // [max_rows * max_chunks], zero between calls
  RowState *states;         // [max_rows]
  StagePartial *partials;   // [max_rows * max_chunks]
  uint32_t max_rows;
  uint32_t max_chunks;
  uint32_t *status;         // device address of a host-mapped word, or NULL
  uint32_t epoch;           // this call's tag (1..4095)
  uint32_t wait_bound;      // reads of a packed best before its wait gives up
  // Room for `rows` drafted rows' stored weights (rows x max_chunks x 8192
  // words), from the owner (called with the upload context), or NULL when
  // the owner keeps none: the residual pass then reads the logits.
  uint32_t *(*lean_weights)(void *ctx, uint32_t rows);
};

// How a selection's host-built row parameters reach scratch.params before
// its kernels run (stream-ordered on `stream`); returns a JF_* status.
typedef int (*ParamUpload)(void *ctx, const RowParams *params, uint32_t rows,
                           RowParams *device, void *stream);

// The body of jf_sample over a given scratch (jf_sampler.cpp): validates the
// call, builds each row's parameters into `params` (host, args->rows
// entries), hands them to `upload`, then enqueues the kernels on `stream`.
// accept: the lanes' tree acceptance to run in the selection's launch if it
// can (*accepted tells whether it did), or NULL.
int sample_core(uint32_t vocabulary, const SampleScratch &scratch,
                const jf_sample_args *args, RowParams *params, ParamUpload upload,
                void *upload_ctx, void *stream, const AcceptTreeLaunch *accept = nullptr,
                bool *accepted = nullptr);

// Launchers (jf_kernels.hip); they return the hipError_t of the launch.
// With both events set, they record the selection kernel's own start and end.
int launch_select(const SampleLaunch &a, uint32_t dtype, void *stream,
                  void *start_event = nullptr, void *stop_event = nullptr);
// `uniform`: when every row of the launch has this policy and penalty table
// row == its own row, or NULL. `fr`: the launch's per-row facts, or NULL for
// a uniform launch with no row map and no extra tokens.
// extras: some row of the launch has extra penalty tokens (fr->row_extra).
// fuse_uncut: every row is sampled with no cut, draft, penalty or extra
// token and no kept outputs are asked for: each row's last chunk block draws
// it (no uncut_kernel launch). accept: the lanes' tree acceptance over this
// launch's rows (greedy lanes, rows = lanes x rows_per_lane), run by the
// row finishers when the launch is uniform, all greedy and finished by
// each row's last chunk; *accepted tells whether it was (else the caller
// launches it).
int launch_select_fast(const FastLaunch &f, const FastRows *fr, uint32_t rows, uint32_t dtype,
                       const RowParams *uniform, bool extras, bool fuse_uncut,
                       const AcceptTreeLaunch *accept, bool *accepted, void *stream,
                       void *start_event = nullptr, void *stop_event = nullptr);
int launch_merge(const SampleLaunch &a, uint32_t dtype, void *stream);
// wide: some cut row of the launch has no min-p floor (longer candidate
// lists); the merge then fetches more list slots a chunk where that helps.
int launch_merge_small(const SampleLaunch &a, uint32_t dtype, bool wide, void *stream);
// Rows with no cut (grid rows x per_row: per_row = chunks when the launch
// has drafted uncut rows, else 1).
int launch_uncut(const SampleLaunch &a, uint32_t dtype, uint32_t per_row, void *stream);
// residual_kernel over the kRowLean rows row_of[0, n_lean) (grid n_lean x
// chunks), before launch_uncut on the same stream; or, with draw set, a
// launch that also draws: each lean row's last chunk block draws that row
// and a share of the rows row_of[n_lean, n_lean + n_plain) (every other row
// of the launch: greedy ones, and sampled ones with no cut, draft, penalty
// or extra token), so no launch_uncut follows (n_lean >= 1, n_lean +
// n_plain <= kKernargRows).
struct LeanLaunch {
  SampleLaunch a;
  uint32_t n_lean;
  uint32_t n_plain;
  uint32_t draw;
  uint32_t row_of[kKernargRows];
};
int launch_residual(const LeanLaunch &l, uint32_t dtype, void *stream);
int launch_stage(const SampleLaunch &a, uint32_t dtype, void *stream);
int launch_accept_chain(const AcceptChainLaunch &a, void *stream);
int launch_accept_tree(const AcceptTreeLaunch &a, void *stream);
// jf_draft.hip; the events, when set, bracket the top-16 kernel.
int launch_draft_select(const DraftLaunch &d, bool aligned, void *stream,
                        void *start_event = nullptr, void *stop_event = nullptr);
// jf_gather.hip; vec8: 8 columns per thread with 16-byte accesses.
int launch_tree_gather(const GatherLaunch &g, bool vec8, void *stream,
                       void *start_event = nullptr, void *stop_event = nullptr);

// The device penalty table as penalty_count_kernel updates it.
struct PenaltyTableView {
  PenaltyEntry *entries;  // [rows][max_entries]
  uint32_t *offsets;      // [rows][buckets + 1]
  uint32_t *slots;        // [rows][chunks][slot_count]
  uint32_t max_entries;
  uint32_t buckets;
  uint32_t chunks;
  uint32_t slot_count;
};

// Up to kPenaltyOps counted tokens (PenaltyOp, packed), in call order within
// each row; block g applies ops [group_start[g], group_start[g + 1]) to
// table row group_row[g].
constexpr uint32_t kPenaltyOps = 64;
struct PackedPenaltyOp {
  uint32_t token;
  uint32_t word;
  uint32_t index;       // entry index | insert << 31
  uint32_t entries;     // the row's entry count before the op
  uint32_t slot_value;
  uint32_t slot;        // slot index | the chunk's used slots << 16; 0xffff: no slot
};
struct PenaltyOpBatch {
  PackedPenaltyOp op[kPenaltyOps];
  uint32_t group_row[kPenaltyOps];
  uint32_t group_start[kPenaltyOps + 1];
};
static_assert(sizeof(PenaltyOpBatch) <= 2560, "penalty updates travel as kernel arguments");

int launch_penalty_count(const PenaltyTableView &t, const PenaltyOpBatch &b, uint32_t groups,
                         void *stream);
// The same updates read from host-mapped memory (calls of more than
// kPenaltyOps tokens, all in one launch): ops[n], group_row[groups],
// group_start[groups + 1].
int launch_penalty_count_mapped(const PenaltyTableView &t, const PackedPenaltyOp *ops,
                                const uint32_t *group_row, const uint32_t *group_start,
                                uint32_t groups, void *stream);

}  // namespace jf
