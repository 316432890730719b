/*
 * jf_oracle — CPU restatement of JustFit's logits->token path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline. The product (libjf_sampler.so) never links,
 * loads or calls it.
 *
 * Every function restates the reference's semantics with sequential, plainly
 * ordered code; the file:line citations point into the reference tree
 * (source/runtime/...). Where the reference's arithmetic is Metal fast-math
 * whose rounding cannot be reproduced off an Apple GPU, this restatement pins
 * one definition that the HIP build must meet bit for bit:
 *   - weights w = jfo_expf((x - M) * inv_t), jfo_expf = Cephes expf (Moshier),
 *     zero below x = -86;
 *   - every sum that decides a token (top-p mass, nucleus walk, the draw, the
 *     residual) runs on w_q = floor(w * 2^44) in exact 64-bit integers, so the
 *     order of summation cannot change a result;
 *   - sampled rows never keep a NaN logit;
 *   - rows with no cut sum per 8192-token chunk against the chunk maximum and
 *     rescale each chunk by jfo_chunk_scale (exp in double by jfo_exp64, a
 *     32-bit significand and a shift).
 * How each function is pinned (brute force, closed form, known answers,
 * statistics) is recorded next to it in jf_oracle.c; nothing here is "parity
 * unpinned".
 */
#ifndef JF_ORACLE_H
#define JF_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JFO_NO_TOKEN 0xffffffffu
#define JFO_PENALTY_PROMPT_BIT 0x80000000u
#define JFO_PENALTY_COUNT_MASK 0x7fffffffu
#define JFO_WEIGHT_BITS 44
#define JFO_DRAFT_CANDIDATES 16u

#define JFO_ROW_CONSTRAINED 1u
#define JFO_ROW_EXCLUDE_STOP 2u

uint32_t jfo_logit_key(float value);
float jfo_key_logit(uint32_t key);
float jfo_expf(float x);
uint64_t jfo_floor_mul(uint64_t a, float f);
uint64_t jfo_residual(uint64_t w, uint64_t mass, float q);
double jfo_exp64(double x);
uint64_t jfo_chunk_scale(float chunk_max, float row_max, float inv_t);
uint64_t jfo_scale_by(uint64_t x, uint64_t scale);
float jfo_uncut_probability(float w, uint64_t scale, uint64_t W);
uint64_t jfo_splitmix64(uint64_t seed, uint64_t counter);
float jfo_next_uniform(uint64_t seed, uint64_t *counter);
void jfo_stage_cycle(uint64_t seed, uint64_t *counter, uint32_t verify_rows,
                     int tree_cycle, float *uniforms40);

int jfo_rebuild_penalty_words(uint32_t *words, uint32_t vocabulary,
                              const uint32_t *history, uint64_t history_len,
                              uint64_t generated, int has_pending,
                              uint32_t pending, int mark_prompt);
int jfo_count_penalty_tokens(uint32_t *words, uint32_t vocabulary,
                             const uint32_t *selected, uint64_t count);
float jfo_penalize_logit(float value, uint32_t count, float repetition,
                         float repetition_inverse, float presence,
                         float frequency);
float jfo_repetition_inverse(float repetition);

typedef struct {
  uint32_t top_k;      /* 0 or >= vocabulary: disabled */
  float temperature;   /* 0: greedy */
  float top_p;         /* (0, 1] */
  float min_p;         /* [0, 1] */
  float repetition;    /* > 0 */
  float presence;
  float frequency;
  uint32_t flags;      /* JFO_ROW_CONSTRAINED | JFO_ROW_EXCLUDE_STOP */
} jfo_policy;

typedef struct {
  const float *logits;          /* fp32 row, or NULL when logits_bf16 is set */
  const uint16_t *logits_bf16;  /* bf16 row (widened exactly) */
  const uint32_t *mask;         /* ceil(V/32) words when constrained */
  const uint32_t *words;        /* dense penalty words [V], or NULL */
  const uint32_t *extra;        /* tokens counted once each on top of words */
  uint32_t extra_count;
  float uniform;
  uint32_t draft_token;         /* JFO_NO_TOKEN: not drafted */
  const uint32_t *cand_ids;     /* sparse q: JFO_DRAFT_CANDIDATES ids */
  const float *cand_probs;      /*           and their probabilities */
  const float *dense_q;         /* dense q [V] (takes precedence) */
} jfo_row_input;

typedef struct {
  uint32_t token;
  float draft_probability;
  uint32_t kept_count;
  float maximum;
} jfo_row_output;

/* Validation of a request's sampling fields (Model.hpp:77-95): 0 if valid. */
int jfo_policy_valid(const jfo_policy *policy);

/* One selected row: greedy argmax or the sampled draw. kept_ids/kept_probs
 * (optional, capacity kept_capacity) receive the kept set in id order. */
int jfo_select_row(uint32_t vocabulary, uint32_t stop0, uint32_t stop1,
                   const jfo_policy *policy, const jfo_row_input *in,
                   jfo_row_output *out, uint32_t *kept_ids, float *kept_probs,
                   uint32_t kept_capacity);

/* Rows of one batch over `threads` host threads (the CPU baseline). Row r
 * reads logits + r * stride (fp32 or bf16 by is_bf16), mask + r * mask_stride,
 * words + pen_row[r] * V when pen_row[r] != JFO_NO_TOKEN, uniforms[r]. */
int jfo_select_batch(uint32_t rows, uint32_t vocabulary, uint32_t stop0,
                     uint32_t stop1, const jfo_policy *policies,
                     const void *logits, int is_bf16, uint64_t stride,
                     const uint32_t *mask, uint64_t mask_stride,
                     const uint32_t *words, const uint32_t *pen_row,
                     const float *uniforms, uint32_t *out_tokens,
                     float *out_maximum, uint32_t threads);

/* Chain acceptance of one lane (sampling.metal:1381-1423, 1514-1558). */
typedef struct {
  uint32_t proposals;        /* verify rows - 1 */
  uint32_t remaining;        /* maximum retained, 1..verify rows */
  uint32_t stop0, stop1;
  int sampled;
} jfo_chain_params;
void jfo_accept_chain(const jfo_chain_params *p, const uint32_t *draft_tokens,
                      const uint32_t *cand_ids, const float *cand_probs,
                      const float *target_draft_prob, const float *uniforms40,
                      uint32_t *target_tokens, uint32_t *retained,
                      uint32_t *accepted);

/* Tree acceptance of one lane (tree.metal:20-84). */
#define JFO_TREE_MAX_ROWS 16u
#define JFO_TREE_MAX_DEPTH 8u
typedef struct {
  uint32_t rows;
  uint32_t chain_rows;
  uint32_t remaining;
  uint32_t stop0, stop1;
  int sampled;
  uint32_t parent[JFO_TREE_MAX_ROWS];
  uint32_t token[JFO_TREE_MAX_ROWS];
  float chain_q[JFO_TREE_MAX_DEPTH];
} jfo_tree_params;
void jfo_accept_tree(const jfo_tree_params *p, const float *target_draft_prob,
                     const float *uniforms40, uint32_t *target_tokens,
                     uint32_t *retained, uint32_t *accepted,
                     uint32_t *path_rows);

/* Draft selector (the DFlash draft's proposal policy: sampling.metal:995-1359,
 * DraftSelector.cpp:38-92). A lane has 8 query rows; rows 1..7 are its
 * proposal positions. */
#define JFO_DRAFT_POSITIONS 7u
#define JFO_DRAFT_QUERY_ROWS 8u
#define JFO_DRAFT_RANK 256u

/* The exact top 16 of one fp32 row in (value desc, id asc) order among its
 * non-NaN tokens (-0 and +0 tie, and tie by id); slots past the row's
 * non-NaN count hold (-inf, JFO_NO_TOKEN) (sampling.metal:995-1013,
 * 1040-1165, 1170-1203). */
void jfo_draft_top16(const float *row, uint32_t vocabulary, uint32_t *ids,
                     float *values);

/* One edge score: the sum over d = 0..255, in that order, of
 * (pred[d] * hidden[d]) * succ[d], bf16 operands widened exactly, fp32
 * products (exact) and fp32 accumulation without contraction
 * (sampling.metal:1249-1288 scores the same sum in another order). */
float jfo_draft_edge(const uint16_t *pred_row, const uint16_t *hidden,
                     const uint16_t *succ_row);

typedef struct {
  uint32_t vocabulary;
  uint32_t anchor;
  float temperature;  /* a sampled lane's */
  int sampled;
} jfo_draft_lane;

/* One lane end to end: candidates and unary scores of its 7 positions, the
 * edge tables, then the walk (sampling.metal:1296-1359). logits8/hidden8 are
 * the lane's 8 query rows (row stride `stride` floats / 256 bf16); uniforms40
 * is the lane's 40 uniforms (position p draws slot 1 + p). q (7 x 16) is
 * written for a sampled lane only. */
void jfo_draft_select_lane(const jfo_draft_lane *lane, const float *logits8,
                           uint64_t stride, const uint16_t *hidden8,
                           const uint16_t *pred_codebook,
                           const uint16_t *succ_codebook,
                           const float *uniforms40, uint32_t *candidates,
                           float *unary, uint32_t *tokens, float *q);

/* Tree gather (verify_tree_gather, tree.metal:86-107; params TreeVerify.h:54-69):
 * for each lane b < lanes, layer y < layers and column c < columns, element
 * (row, c) sits at base + row * row_stride with base = y * layer_stride +
 * b * lane_stride + (c / inner) * outer_stride + (c % inner) * inner_stride
 * (16-bit units); rows i < retained[b] take row path_rows[b * 8 + i], copied
 * in increasing i, in place. Sources at or past `rows` (rows per lane) are
 * skipped. */
typedef struct {
  uint32_t columns, inner, inner_stride, outer_stride, row_stride, lane_stride,
      layer_stride, layers, lanes, rows;
} jfo_gather_params;
void jfo_tree_gather(uint16_t *data, const uint32_t *path_rows,
                     const uint32_t *retained, const jfo_gather_params *p);

#ifdef __cplusplus
}
#endif
#endif
