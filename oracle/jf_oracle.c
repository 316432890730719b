/*
 * jf_oracle.c — CPU restatement of JustFit's logits->token path.
 *
 * TEST INFRASTRUCTURE ONLY (see jf_oracle.h): the checker for the HIP build
 * and the timed CPU baseline. Built with -O2 -ffp-contract=off so every fp32
 * expression rounds exactly as written.
 *
 * Pins (tests/test_oracle.py):
 *   jfo_logit_key / jfo_key_logit  order and +-0 against float compares,
 *                                  round trip over sampled bit patterns.
 *   jfo_expf                       <= 2 ulp against double exp over a sweep.
 *   jfo_floor_mul                  against Python's exact integers.
 *   jfo_residual                   against numpy float32 products and
 *                                  Python integers, with the NaN, sign,
 *                                  2^32 and 2^44 edges.
 *   jfo_splitmix64                 published SplitMix64 known answers
 *                                  (Steele, Lea & Flood 2014; seed 0 ->
 *                                  0xe220a8397b1dcdaf).
 *   penalty words                  against a dict-based restatement and the
 *                                  closed-form penalty formula.
 *   jfo_select_row greedy          np.argmax with lowest-id ties.
 *   jfo_select_row sampled         brute force over tiny vocabularies
 *                                  (itertools/fractions), kept sets against
 *                                  sort-by-(logit desc, id asc), probabilities
 *                                  against float64 softmax (1e-5), chi-square
 *                                  of the draw over many uniforms, and the
 *                                  speculative-sampling identity for the
 *                                  residual draw.
 *   chain/tree acceptance          hand-built cases, chain-shaped trees equal
 *                                  to chain acceptance.
 */
#include "jf_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---- scalar helpers --------------------------------------------------- */

static uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* sampling.metal:167-171: a larger logit has a larger key; -0 and +0 share. */
uint32_t jfo_logit_key(float value) {
  uint32_t bits = f2u(value);
  bits = (bits << 1) ? bits : 0u;
  return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

/* sampling.metal:172-174 */
float jfo_key_logit(uint32_t key) {
  return u2f((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

/* Cephes expf (S. L. Moshier, Cephes Math Library): x = n ln2 + r with the
 * two-constant Cody-Waite split of ln2, e^r = 1 + r + r^2 P(r) with Cephes'
 * degree-5 P, then scaling by 2^n. Below -86 the result is 0, so every
 * nonzero result is a normal float. */
float jfo_expf(float x) {
  if (!(x >= -86.0f))
    return 0.0f;
  if (x > 88.0f)
    return INFINITY;
  const float n = rintf(x * 1.44269504088896341f);
  float r = fmaf(n, -0.693359375f, x);
  r = fmaf(n, 2.12194440e-4f, r);
  float p = 1.9875691500e-4f;
  p = fmaf(p, r, 1.3981999507e-3f);
  p = fmaf(p, r, 8.3334519073e-3f);
  p = fmaf(p, r, 4.1665795894e-2f);
  p = fmaf(p, r, 1.6666665459e-1f);
  p = fmaf(p, r, 5.0000001201e-1f);
  const float r2 = r * r;
  const float y = fmaf(p, r2, r) + 1.0f;
  const int ni = (int)n;
  return y * u2f((uint32_t)(ni + 127) << 23);
}

/* e^x in double, for the per-chunk rescale of rows with no cut: the Cody-Waite
 * reduction x = n ln2 + r (n = rint(x log2 e), ln2 split into a 28-bit head,
 * so n * head is exact, and the rounded rest), |r| <= ln2 / 2, then e^r by its
 * Taylor series to degree 13 (the truncation is below 5e-18 relative) in
 * Horner form with fused multiply-adds, times 2^n. Every step is one IEEE
 * double operation, so the device restatement gives the same bits. Zero below
 * -708 (where 2^n would leave the normal range) and for NaN. */
double jfo_exp64(double x) {
  if (!(x >= -708.0))
    return 0.0;
  if (x > 709.0)
    return INFINITY;
  const double n = rint(x * 0x1.71547652b82fep+0);
  double r = fma(n, -0x1.62e42ffp-1, x);
  r = fma(n, 0x1.718432a1b0e26p-35, r);
  double p = 0x1.6124613a86d09p-33;  /* 1/13! */
  p = fma(p, r, 0x1.1eed8eff8d898p-29);
  p = fma(p, r, 0x1.ae64567f544e4p-26);
  p = fma(p, r, 0x1.27e4fb7789f5cp-22);
  p = fma(p, r, 0x1.71de3a556c734p-19);
  p = fma(p, r, 0x1.a01a01a01a01ap-16);
  p = fma(p, r, 0x1.a01a01a01a01ap-13);
  p = fma(p, r, 0x1.6c16c16c16c17p-10);
  p = fma(p, r, 0x1.1111111111111p-7);
  p = fma(p, r, 0x1.5555555555555p-5);
  p = fma(p, r, 0x1.5555555555555p-3);
  p = fma(p, r, 0x1p-1);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  const uint64_t bits = (uint64_t)((int64_t)n + 1023) << 52;
  double two_n;
  memcpy(&two_n, &bits, 8);
  return p * two_n;
}

/* The rescale of a chunk's mass from its maximum m_c to the row maximum M:
 * r = exp64((m_c - M) * inv_t) (the difference and product in double) as
 * R * 2^-s, R its 53-bit significand rounded (half up) to 32 bits, so R is in
 * [2^31, 2^32) and the relative error of the representation is at most
 * 2^-32 whatever the offset. r = 0 gives R = 0, s = 64. Returned packed as
 * s << 32 | R (the kernels keep it in one 64-bit word). */
uint64_t jfo_chunk_scale(float chunk_max, float row_max, float inv_t) {
  const double r = jfo_exp64(((double)chunk_max - (double)row_max) * (double)inv_t);
  if (!(r > 0.0))
    return 64ull << 32;
  uint64_t bits;
  memcpy(&bits, &r, 8);
  const int e = (int)(bits >> 52) - 1023;  /* r normal: e in [-1022, 0] */
  uint64_t R = (((bits & 0xfffffffffffffull) | (1ull << 52)) + (1ull << 20)) >> 21;
  uint64_t s = (uint64_t)(31 - e);
  if (R >> 32) {
    R >>= 1;
    s -= 1;
  }
  return s << 32 | R;
}

/* floor(x * R * 2^-s) exactly, for the packed rescale s << 32 | R. */
uint64_t jfo_scale_by(uint64_t x, uint64_t scale) {
  const uint64_t R = scale & 0xffffffffull, s = scale >> 32;
  if (s >= 128)
    return 0;
  return (uint64_t)(((unsigned __int128)x * R) >> s);
}

/* A token's reported probability on a row with no cut: its float weight w
 * against its chunk's maximum, times the chunk's rescale, over the row mass
 * W (units of 2^-44), in double; results below FLT_MIN report 0 (on both
 * sides of the build, so no denormal conversion is involved). */
float jfo_uncut_probability(float w, uint64_t scale, uint64_t W) {
  if (!W)
    return 0.0f;
  const uint64_t R = scale & 0xffffffffull, s = scale >> 32;
  const double r = ldexp((double)R, -(int)s);
  const double p = ((double)w * r) / ((double)W * 0x1p-44);
  return p >= (double)FLT_MIN ? (float)p : 0.0f;
}

/* A drafted row's residual weight max(w - Q, 0) (sampling.metal:700-708,
 * 760-765): Q = floor(q * m) for m the mass rounded to a float and the
 * product rounded to a float (both to nearest even, as the kernels compute
 * it). q NaN or <= 0 gives Q = 0; Q at or above 2^44 leaves nothing, since
 * every weight is at most 2^44. */
uint64_t jfo_residual(uint64_t w, uint64_t mass, float q) {
  const float m = (float)mass;
  const float x = q > 0.0f ? q * m : 0.0f;
  if (!(x < 0x1p44f))
    return 0;
  const uint64_t qm = (uint64_t)x;
  return w > qm ? w - qm : 0;
}

/* floor(a * f) exactly, for f in [0, 1] (NaN and f <= 0 give 0, f >= 1 gives
 * a). f = M * 2^-sh with a 24-bit M, so the product fits 128 bits. */
uint64_t jfo_floor_mul(uint64_t a, float f) {
  if (!(f > 0.0f))
    return 0;
  if (f >= 1.0f)
    return a;
  const uint32_t b = f2u(f);
  const uint32_t e = b >> 23;
  const uint64_t m = e ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu);
  const int sh = e ? 150 - (int)e : 149;
  const unsigned __int128 p = (unsigned __int128)a * m;
  return sh >= 128 ? 0 : (uint64_t)(p >> sh);
}

/* Runtime.cpp:1098-1105 (SplitMix64 finalizer over seed + counter * golden). */
uint64_t jfo_splitmix64(uint64_t seed, uint64_t counter) {
  uint64_t v = seed + counter * 0x9e3779b97f4a7c15ULL;
  v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
  v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
  return v ^ (v >> 31);
}

float jfo_next_uniform(uint64_t seed, uint64_t *counter) {
  const uint64_t v = jfo_splitmix64(seed, ++*counter);
  return (float)(v >> 40) * 0x1p-24f;
}

/* Runtime.cpp:1107-1114: slots 1.. of a cycle; 16 for 8 verify rows, 24 for
 * 16, all 40 for a 16-row tree cycle. */
void jfo_stage_cycle(uint64_t seed, uint64_t *counter, uint32_t verify_rows,
                     int tree_cycle, float *u) {
  for (int i = 0; i < 40; ++i)
    u[i] = 0.0f;
  const uint32_t end =
      (tree_cycle && verify_rows == 16) ? 40u : verify_rows == 16 ? 24u : 16u;
  for (uint32_t i = 1; i < end; ++i)
    u[i] = jfo_next_uniform(seed, counter);
}

/* ---- penalties -------------------------------------------------------- */

/* Sampling.cpp:50-71 (rebuildPenaltyWords). Returns -1 for a history without
 * a prompt, -2 for a token outside the vocabulary. */
int jfo_rebuild_penalty_words(uint32_t *words, uint32_t vocabulary,
                              const uint32_t *history, uint64_t history_len,
                              uint64_t generated, int has_pending,
                              uint32_t pending, int mark_prompt) {
  if (history_len <= generated)
    return -1;
  for (uint64_t i = 0; i < history_len; ++i)
    if (history[i] >= vocabulary)
      return -2;
  if (has_pending && pending >= vocabulary)
    return -2;
  const uint64_t prompt = history_len - generated;
  memset(words, 0, (size_t)vocabulary * 4);
  if (mark_prompt)
    for (uint64_t i = 0; i < prompt; ++i)
      words[history[i]] |= JFO_PENALTY_PROMPT_BIT;
  for (uint64_t i = prompt; i < history_len; ++i)
    ++words[history[i]];
  if (has_pending)
    ++words[pending];
  return 0;
}

/* Sampling.cpp:75-80 (countPenaltyTokens). */
int jfo_count_penalty_tokens(uint32_t *words, uint32_t vocabulary,
                             const uint32_t *selected, uint64_t count) {
  for (uint64_t i = 0; i < count; ++i)
    if (selected[i] >= vocabulary)
      return -2;
  for (uint64_t i = 0; i < count; ++i)
    ++words[selected[i]];
  return 0;
}

/* Sampling.cpp:110-112: 1 / repetition, saturated to the largest float. */
float jfo_repetition_inverse(float repetition) {
  const float inv = 1.0f / repetition;
  return inv < FLT_MAX ? inv : FLT_MAX;
}

/* sampling.metal:928-935 (penalize_logit); clamp = fmin(fmax(.)), so a NaN
 * becomes -FLT_MAX. */
float jfo_penalize_logit(float value, uint32_t count, float repetition,
                         float repetition_inverse, float presence,
                         float frequency) {
  value *= value > 0.0f ? repetition_inverse : repetition;
  if (count) {
    const float scaled = frequency * (float)count;
    const float lowered = scaled + presence;
    value = value - lowered;
  }
  return fminf(fmaxf(value, -FLT_MAX), FLT_MAX);
}

/* ---- policy ----------------------------------------------------------- */

/* Model.hpp:77-95 (validationError). */
int jfo_policy_valid(const jfo_policy *p) {
  const int t_ok = p->temperature == 0.0f ||
                   (isfinite(p->temperature) && p->temperature >= FLT_MIN);
  if (!t_ok || !(p->top_p > 0.0f && p->top_p <= 1.0f) || !(p->min_p >= 0.0f) ||
      p->min_p > 1.0f)
    return -1;
  if (!(fabsf(p->presence) <= 2.0f) || !(fabsf(p->frequency) <= 2.0f) ||
      !isfinite(p->repetition) || p->repetition <= 0.0f)
    return -2;
  return 0;
}

static int penalties_active(const jfo_policy *p) {
  return p->repetition != 1.0f || p->presence != 0.0f || p->frequency != 0.0f;
}

/* ---- one row ---------------------------------------------------------- */

typedef struct {
  uint32_t key;
  uint32_t id;
} keyed;

/* Order of the logits: key descending, id ascending (sampling.metal:176-207). */
static int by_order(const void *a, const void *b) {
  const keyed *x = (const keyed *)a, *y = (const keyed *)b;
  if (x->key != y->key)
    return x->key > y->key ? -1 : 1;
  return x->id < y->id ? -1 : (x->id > y->id);
}
static int by_id(const void *a, const void *b) {
  const keyed *x = (const keyed *)a, *y = (const keyed *)b;
  return x->id < y->id ? -1 : (x->id > y->id);
}

static float row_value(const jfo_row_input *in, uint32_t t) {
  if (in->logits)
    return in->logits[t];
  return u2f((uint32_t)in->logits_bf16[t] << 16);
}

/* TargetRow::admits (sampling.metal:33-37). */
static int admits(const jfo_policy *p, const jfo_row_input *in, uint32_t t,
                  uint32_t stop0, uint32_t stop1) {
  if ((p->flags & JFO_ROW_CONSTRAINED) &&
      !(in->mask[t / 32] & (1u << (t % 32))))
    return 0;
  return !(p->flags & JFO_ROW_EXCLUDE_STOP) || (t != stop0 && t != stop1);
}

/* The row's logit of token t after its penalties (sampling.metal:941-963;
 * Sampling.cpp:88-132): only rows whose policy has active penalties. */
static float penalized(const jfo_policy *p, float inv_rep,
                       const jfo_row_input *in, uint32_t t) {
  float v = row_value(in, t);
  if (!penalties_active(p))
    return v;
  const uint32_t word = in->words ? in->words[t] : 0u;
  uint32_t count = word & JFO_PENALTY_COUNT_MASK;
  for (uint32_t i = 0; i < in->extra_count; ++i)
    count += in->extra[i] == t;
  if (!count && !(word & JFO_PENALTY_PROMPT_BIT))
    return v;
  return jfo_penalize_logit(v, count, p->repetition, inv_rep, p->presence,
                            p->frequency);
}

/* The draft's probability of token t: dense q, or the first of the sparse
 * candidates that lists t (sampling.metal:703-708, 1361-1369). */
static float draft_q(const jfo_row_input *in, uint32_t t) {
  if (in->dense_q)
    return in->dense_q[t];
  if (!in->cand_ids)
    return 0.0f;
  for (uint32_t j = 0; j < JFO_DRAFT_CANDIDATES; ++j)
    if (in->cand_ids[j] == t)
      return in->cand_probs[j];
  return 0.0f;
}

static uint64_t quantize(float w) {
  return (uint64_t)(w * 0x1p44f);
}

/* ---- rows that keep every admitted token ------------------------------ */

/* A sampled row with no min-p, top-k or top-p cut keeps every admitted
 * token. Its mass is exact per 8192-token chunk c against the chunk's own
 * maximum m_c,
 *   S_c = sum over the chunk of quantize(expf((x - m_c) / T)),
 * and each chunk's mass is rescaled to the row maximum M once, by
 * r_c = exp((m_c - M) / T) carried as R_c * 2^-s_c (jfo_chunk_scale: a 32-bit
 * significand, relative precision 2^-32 at any offset):
 *   T_c = floor(S_c * r_c),   W = sum of T_c.
 * The draw takes u * W, the chunk whose running T_c passes it, and inside
 * that chunk the first token (id order) whose running S-mass P satisfies
 * floor(P * r_c) > the remainder. A drafted row draws the residual
 * max(floor(w_q * r_c) - floor(W * q), 0) in id order (w_q the token's
 * quantized weight), or plainly when no residual mass remains
 * (sampling.metal:694-829 on these weights). A token's reported probability
 * (kept outputs, p(draft)) is its float weight times r_c over the mass,
 * float(w * r_c / (W * 2^-44)) in double (jfo_uncut_probability), which is
 * exp((x - M) / T) / sum to float precision at any offset down to where float
 * results underflow. One pass over the logits yields every S_c, so the GPU
 * reads the row once. With a single chunk (V <= 8192) r = 1 and this is the
 * row-maximum definition. */
#define JFO_MASS_CHUNK 8192u

static int uncut_select(uint32_t V, uint32_t stop0, uint32_t stop1,
                        const jfo_policy *p, float inv_rep, float inv_t,
                        const jfo_row_input *in, float M, uint32_t n,
                        jfo_row_output *out, uint32_t *kept_ids,
                        float *kept_probs, uint32_t kept_capacity) {
  const uint32_t C = (V + JFO_MASS_CHUNK - 1) / JFO_MASS_CHUNK;
  float *cmax = (float *)malloc(sizeof(float) * C);
  uint64_t *cmass = (uint64_t *)calloc(C, sizeof(uint64_t));
  uint64_t *cscale = (uint64_t *)malloc(sizeof(uint64_t) * C);
  uint64_t *ctot = (uint64_t *)malloc(sizeof(uint64_t) * C);
  if (!cmax || !cmass || !cscale || !ctot) {
    free(cmax); free(cmass); free(cscale); free(ctot);
    return -3;
  }
  for (uint32_t c = 0; c < C; ++c)
    cmax[c] = -FLT_MAX;
  for (uint32_t t = 0; t < V; ++t) {
    if (!admits(p, in, t, stop0, stop1))
      continue;
    const float v = penalized(p, inv_rep, in, t);
    if (v > cmax[t / JFO_MASS_CHUNK])
      cmax[t / JFO_MASS_CHUNK] = v;
  }
  for (uint32_t t = 0; t < V; ++t) {
    if (!admits(p, in, t, stop0, stop1))
      continue;
    const float v = penalized(p, inv_rep, in, t);
    if (!isnan(v))
      cmass[t / JFO_MASS_CHUNK] += quantize(jfo_expf((v - cmax[t / JFO_MASS_CHUNK]) * inv_t));
  }
  uint64_t W = 0;
  for (uint32_t c = 0; c < C; ++c) {
    cscale[c] = jfo_chunk_scale(cmax[c], M, inv_t);
    ctot[c] = jfo_scale_by(cmass[c], cscale[c]);
    W += ctot[c];
  }
  /* The kept set is every admitted non-NaN token, in id order. */
  out->kept_count = n;
  #define FLOAT_WEIGHT(t, v) jfo_expf(((v) - cmax[(t) / JFO_MASS_CHUNK]) * inv_t)
  #define WEIGHT_OF(t, v) quantize(FLOAT_WEIGHT(t, v))
  #define PROB_OF(t, v) \
    jfo_uncut_probability(FLOAT_WEIGHT(t, v), cscale[(t) / JFO_MASS_CHUNK], W)
  if (kept_ids) {
    uint32_t k = 0;
    for (uint32_t t = 0; t < V && k < kept_capacity; ++t) {
      if (!admits(p, in, t, stop0, stop1))
        continue;
      const float v = penalized(p, inv_rep, in, t);
      if (isnan(v))
        continue;
      kept_ids[k] = t;
      kept_probs[k] = PROB_OF(t, v);
      ++k;
    }
  }
  const int drafted = in->draft_token != JFO_NO_TOKEN;
  if (W != 0) {
    int drawn = 0;
    if (drafted) {
      /* The residual weights (jfo_residual) in id order. */
      uint64_t total = 0;
      for (uint32_t t = 0; t < V; ++t) {
        if (!admits(p, in, t, stop0, stop1))
          continue;
        const float v = penalized(p, inv_rep, in, t);
        if (isnan(v))
          continue;
        const uint64_t w = jfo_scale_by(WEIGHT_OF(t, v), cscale[t / JFO_MASS_CHUNK]);
        total += jfo_residual(w, W, draft_q(in, t));
      }
      if (total) {
        uint64_t target = jfo_floor_mul(total, in->uniform);
        if (target >= total)
          target = total - 1;
        uint64_t run = 0;
        for (uint32_t t = 0; t < V && !drawn; ++t) {
          if (!admits(p, in, t, stop0, stop1))
            continue;
          const float v = penalized(p, inv_rep, in, t);
          if (isnan(v))
            continue;
          const uint64_t w = jfo_scale_by(WEIGHT_OF(t, v), cscale[t / JFO_MASS_CHUNK]);
          run += jfo_residual(w, W, draft_q(in, t));
          if (run > target) {
            out->token = t;
            drawn = 1;
          }
        }
      }
    }
    if (!drawn) {
      uint64_t target = jfo_floor_mul(W, in->uniform);
      if (target >= W)
        target = W - 1;
      uint32_t c = 0;
      uint64_t before = 0;
      while (before + ctot[c] <= target)
        before += ctot[c++];
      const uint64_t within = target - before;
      uint64_t P = 0;
      const uint32_t end = (c + 1) * JFO_MASS_CHUNK < V ? (c + 1) * JFO_MASS_CHUNK : V;
      for (uint32_t t = c * JFO_MASS_CHUNK; t < end; ++t) {
        if (!admits(p, in, t, stop0, stop1))
          continue;
        const float v = penalized(p, inv_rep, in, t);
        if (isnan(v))
          continue;
        P += WEIGHT_OF(t, v);
        if (jfo_scale_by(P, cscale[c]) > within) {
          out->token = t;
          break;
        }
      }
    }
    /* p(draft) (sampling.metal:828-829). */
    const uint32_t d = in->draft_token;
    if (drafted && d < V && admits(p, in, d, stop0, stop1)) {
      const float v = penalized(p, inv_rep, in, d);
      if (!isnan(v))
        out->draft_probability = PROB_OF(d, v);
    }
  }
  #undef PROB_OF
  #undef WEIGHT_OF
  #undef FLOAT_WEIGHT
  free(cmax); free(cmass); free(cscale); free(ctot);
  return 0;
}

int jfo_select_row(uint32_t V, uint32_t stop0, uint32_t stop1,
                   const jfo_policy *p, const jfo_row_input *in,
                   jfo_row_output *out, uint32_t *kept_ids, float *kept_probs,
                   uint32_t kept_capacity) {
  const float inv_rep = jfo_repetition_inverse(p->repetition);
  out->token = JFO_NO_TOKEN;
  out->draft_probability = 0.0f;
  out->kept_count = 0;
  out->maximum = -FLT_MAX;

  /* Greedy (sampling.metal:1427-1512): admitted argmax, largest value then
   * lowest id; NaN never wins; a -inf row gives its lowest admitted id. */
  if (!(p->temperature > 0.0f)) {
    float best = -INFINITY;
    uint32_t best_id = JFO_NO_TOKEN;
    for (uint32_t t = 0; t < V; ++t) {
      if (!admits(p, in, t, stop0, stop1))
        continue;
      const float v = penalized(p, inv_rep, in, t);
      if (v > best || (v == best && t < best_id)) {
        best = v;
        best_id = t;
      }
    }
    out->token = best_id;
    out->maximum = best;
    return 0;
  }

  /* Sampled. The admitted non-NaN tokens, their maximum M
   * (sampling.metal:95-127 keeps -inf out of M). */
  keyed *list = (keyed *)malloc(sizeof(keyed) * (V ? V : 1));
  if (!list)
    return -3;
  uint32_t n = 0;
  float M = -FLT_MAX;
  for (uint32_t t = 0; t < V; ++t) {
    if (!admits(p, in, t, stop0, stop1))
      continue;
    const float v = penalized(p, inv_rep, in, t);
    if (isnan(v))
      continue;
    if (v > M)
      M = v;
    list[n].key = jfo_logit_key(v);
    list[n].id = t;
    ++n;
  }
  out->maximum = M;
  if (n == 0 || M == INFINITY) {
    free(list);
    return 0;
  }
  const float inv_t = 1.0f / p->temperature;
  if (!(p->min_p > 0.0f) && !(p->top_k && p->top_k < V) && !(p->top_p < 1.0f)) {
    free(list);
    return uncut_select(V, stop0, stop1, p, inv_rep, inv_t, in, M, n, out, kept_ids,
                        kept_probs, kept_capacity);
  }
  qsort(list, n, sizeof(keyed), by_order);

  /* min-p (sampling.metal:593-607): keys at or above that of
   * min(M + T log(min_p), M). */
  uint32_t n1 = n;
  if (p->min_p > 0.0f) {
    const float offset = p->temperature * logf(p->min_p);
    const float floor_value = fminf(M + offset, M);
    const uint32_t floor_key = jfo_logit_key(floor_value);
    n1 = 0;
    while (n1 < n && list[n1].key >= floor_key)
      ++n1;
  }
  /* top-k of those, exactly k in order (sampling.metal:608-637). */
  const uint32_t k_eff = (p->top_k && p->top_k < V) ? p->top_k : V;
  const uint32_t n2 = k_eff < n1 ? k_eff : n1;

  uint64_t *wq = (uint64_t *)malloc(sizeof(uint64_t) * (n2 ? n2 : 1));
  float *w = (float *)malloc(sizeof(float) * (n2 ? n2 : 1));
  if (!wq || !w) {
    free(list);
    free(wq);
    free(w);
    return -3;
  }
  uint64_t mass2 = 0;
  for (uint32_t i = 0; i < n2; ++i) {
    const float x = jfo_key_logit(list[i].key);
    const float d = x - M;
    w[i] = jfo_expf(d * inv_t);
    wq[i] = quantize(w[i]);
    mass2 += wq[i];
  }
  /* top-p over the mass of what min-p and top-k keep: walk in order until
   * the running mass exceeds top_p of it; keep all if it never does
   * (sampling.metal:615-641). */
  uint32_t n3 = n2;
  if (p->top_p < 1.0f) {
    const uint64_t nucleus = jfo_floor_mul(mass2, p->top_p);
    uint64_t walked = 0;
    for (uint32_t i = 0; i < n2; ++i) {
      walked += wq[i];
      if (walked > nucleus) {
        n3 = i + 1;
        break;
      }
    }
  }
  /* The kept set in id order (sampling.metal:645-651). */
  keyed *kept = (keyed *)malloc(sizeof(keyed) * (n3 ? n3 : 1));
  float *kw = (float *)malloc(sizeof(float) * (n3 ? n3 : 1));
  uint64_t *kq = (uint64_t *)malloc(sizeof(uint64_t) * (n3 ? n3 : 1));
  uint64_t *dq = (uint64_t *)malloc(sizeof(uint64_t) * (n3 ? n3 : 1));
  if (!kept || !kw || !kq || !dq) {
    free(list); free(wq); free(w); free(kept); free(kw); free(kq); free(dq);
    return -3;
  }
  for (uint32_t i = 0; i < n3; ++i)
    kept[i] = list[i];
  qsort(kept, n3, sizeof(keyed), by_id);
  uint64_t mass3 = 0;
  for (uint32_t i = 0; i < n3; ++i) {
    const float x = jfo_key_logit(kept[i].key);
    kw[i] = jfo_expf((x - M) * inv_t);
    kq[i] = quantize(kw[i]);
    mass3 += kq[i];
  }
  out->kept_count = n3;
  const double scale = (double)mass3 * 0x1p-44;
  if (kept_ids)
    for (uint32_t i = 0; i < n3 && i < kept_capacity; ++i) {
      kept_ids[i] = kept[i].id;
      kept_probs[i] = mass3 ? (float)((double)kw[i] / scale) : 0.0f;
    }
  if (mass3 == 0) {
    free(list); free(wq); free(w); free(kept); free(kw); free(kq); free(dq);
    return 0;
  }
  /* Draw weights: a drafted row's residual max(w - q * mass, 0), or w when
   * nothing remains of it (sampling.metal:739-765). */
  const int drafted = in->draft_token != JFO_NO_TOKEN;
  int residual = 0;
  for (uint32_t i = 0; i < n3; ++i) {
    if (drafted) {
      dq[i] = jfo_residual(kq[i], mass3, draft_q(in, kept[i].id));
      residual |= dq[i] > 0;
    } else {
      dq[i] = kq[i];
    }
  }
  if (drafted && !residual)
    for (uint32_t i = 0; i < n3; ++i)
      dq[i] = kq[i];
  uint64_t total = 0;
  for (uint32_t i = 0; i < n3; ++i)
    total += dq[i];
  /* Inverse CDF in id order: the first token whose running weight exceeds
   * u * total (sampling.metal:766-829). */
  uint64_t target = jfo_floor_mul(total, in->uniform);
  if (target >= total)
    target = total - 1;
  uint64_t run = 0;
  for (uint32_t i = 0; i < n3; ++i) {
    run += dq[i];
    if (run > target) {
      out->token = kept[i].id;
      break;
    }
  }
  /* p(draft) = kept weight / kept mass (sampling.metal:828-829). */
  if (drafted)
    for (uint32_t i = 0; i < n3; ++i)
      if (kept[i].id == in->draft_token)
        out->draft_probability = (float)((double)kw[i] / scale);
  free(list); free(wq); free(w); free(kept); free(kw); free(kq); free(dq);
  return 0;
}

/* ---- batch over host threads ------------------------------------------ */

typedef struct {
  uint32_t rows, V, stop0, stop1;
  const jfo_policy *policies;
  const void *logits;
  int is_bf16;
  uint64_t stride;
  const uint32_t *mask;
  uint64_t mask_stride;
  const uint32_t *words;
  const uint32_t *pen_row;
  const float *uniforms;
  uint32_t *out_tokens;
  float *out_maximum;
  uint32_t next;
  pthread_mutex_t lock;
  int status;
} batch_job;

static void *batch_worker(void *arg) {
  batch_job *job = (batch_job *)arg;
  for (;;) {
    pthread_mutex_lock(&job->lock);
    const uint32_t r = job->next++;
    pthread_mutex_unlock(&job->lock);
    if (r >= job->rows)
      return NULL;
    jfo_row_input in;
    memset(&in, 0, sizeof(in));
    if (job->is_bf16)
      in.logits_bf16 = (const uint16_t *)job->logits + r * job->stride;
    else
      in.logits = (const float *)job->logits + r * job->stride;
    in.mask = job->mask ? job->mask + r * job->mask_stride : NULL;
    if (job->words && job->pen_row && job->pen_row[r] != JFO_NO_TOKEN)
      in.words = job->words + (uint64_t)job->pen_row[r] * job->V;
    in.uniform = job->uniforms ? job->uniforms[r] : 0.0f;
    in.draft_token = JFO_NO_TOKEN;
    jfo_row_output out;
    const int rc = jfo_select_row(job->V, job->stop0, job->stop1,
                                  &job->policies[r], &in, &out, NULL, NULL, 0);
    if (rc)
      job->status = rc;
    job->out_tokens[r] = out.token;
    if (job->out_maximum)
      job->out_maximum[r] = out.maximum;
  }
}

int jfo_select_batch(uint32_t rows, uint32_t V, uint32_t stop0, uint32_t stop1,
                     const jfo_policy *policies, const void *logits,
                     int is_bf16, uint64_t stride, const uint32_t *mask,
                     uint64_t mask_stride, const uint32_t *words,
                     const uint32_t *pen_row, const float *uniforms,
                     uint32_t *out_tokens, float *out_maximum,
                     uint32_t threads) {
  batch_job job = {rows, V, stop0, stop1, policies, logits, is_bf16, stride,
                   mask, mask_stride, words, pen_row, uniforms, out_tokens,
                   out_maximum, 0, PTHREAD_MUTEX_INITIALIZER, 0};
  if (threads < 1)
    threads = 1;
  if (threads > 256)
    threads = 256;
  pthread_t tid[256];
  uint32_t started = 0;
  for (uint32_t i = 1; i < threads; ++i)
    if (pthread_create(&tid[started], NULL, batch_worker, &job) == 0)
      ++started;
  batch_worker(&job);
  for (uint32_t i = 0; i < started; ++i)
    pthread_join(tid[i], NULL);
  return job.status;
}

/* ---- acceptance ------------------------------------------------------- */

/* finish_acceptance (sampling.metal:1381-1392). */
static void finish(const uint32_t *tokens, uint32_t accepted, uint32_t remaining,
                   uint32_t stop0, uint32_t stop1, uint32_t *retained,
                   uint32_t *accepted_out) {
  *accepted_out = accepted;
  uint32_t kept = accepted + 1 < remaining ? accepted + 1 : remaining;
  for (uint32_t i = 0; i < kept; ++i)
    if (tokens[i] == stop0 || tokens[i] == stop1) {
      kept = i + 1;
      break;
    }
  *retained = kept;
}

/* decode_accept_dflash (sampling.metal:1399-1423, 1514-1558). Acceptance
 * uniform of proposal i: slot 8 + i below 7, slot 16 + i - 7 after. */
void jfo_accept_chain(const jfo_chain_params *p, const uint32_t *draft_tokens,
                      const uint32_t *cand_ids, const float *cand_probs,
                      const float *target_draft_prob, const float *u,
                      uint32_t *target_tokens, uint32_t *retained,
                      uint32_t *accepted_out) {
  uint32_t accepted = 0;
  if (p->sampled) {
    while (accepted < p->proposals) {
      const uint32_t token = draft_tokens[accepted];
      if (token == JFO_NO_TOKEN)
        break;
      float q = 0.0f;
      for (uint32_t j = 0; j < JFO_DRAFT_CANDIDATES; ++j)
        if (cand_ids[accepted * JFO_DRAFT_CANDIDATES + j] == token) {
          q = cand_probs[accepted * JFO_DRAFT_CANDIDATES + j];
          break;
        }
      const float pr = target_draft_prob[accepted];
      const float uu = u[accepted < 7 ? 8 + accepted : 16 + accepted - 7];
      if (!(uu * q < pr))
        break;
      target_tokens[accepted] = token;
      ++accepted;
    }
  } else {
    while (accepted < p->proposals &&
           draft_tokens[accepted] == target_tokens[accepted])
      ++accepted;
  }
  finish(target_tokens, accepted, p->remaining, p->stop0, p->stop1, retained,
         accepted_out);
}

/* verify_tree_accept (tree.metal:20-84). */
void jfo_accept_tree(const jfo_tree_params *p, const float *target_draft_prob,
                     const float *u, uint32_t *tokens, uint32_t *retained,
                     uint32_t *accepted_out, uint32_t *path_rows) {
  uint32_t path[JFO_TREE_MAX_DEPTH];
  uint32_t length = 1, current = 0;
  path[0] = 0;
  while (length < JFO_TREE_MAX_DEPTH) {
    if (p->sampled && current + 1 < p->chain_rows) {
      const float q = p->chain_q[current];
      const float pr = target_draft_prob[current];
      if (u[8 + current] * q < pr) {
        path[length++] = current + 1;
        current = current + 1;
        continue;
      }
    }
    const uint32_t wanted = tokens[current];
    uint32_t found = 0;
    for (uint32_t row = current + 1; row < p->rows; ++row)
      if (p->parent[row] == current && p->token[row] == wanted &&
          !(p->sampled && row == current + 1 && current + 1 < p->chain_rows)) {
        found = row;
        break;
      }
    if (!found)
      break;
    path[length++] = found;
    current = found;
  }
  uint32_t output[JFO_TREE_MAX_DEPTH];
  for (uint32_t i = 0; i < length; ++i)
    output[i] = i + 1 < length ? p->token[path[i + 1]] : tokens[path[i]];
  for (uint32_t i = 0; i < length; ++i)
    tokens[i] = output[i];
  finish(tokens, length - 1, p->remaining, p->stop0, p->stop1, retained,
         accepted_out);
  for (uint32_t i = 0; i < JFO_TREE_MAX_DEPTH; ++i)
    path_rows[i] = i < length ? path[i] : path[length - 1];
}

/* ---- draft selector ---------------------------------------------------- */

/* (value desc, id asc): sampling.metal:995-997. NaN never beats anything. */
static int draft_beats(float v, uint32_t id, float w, uint32_t wid) {
  return v > w || (v == w && id < wid);
}

/* Pinned by tests/test_oracle.py against a numpy lexsort over random rows,
 * rows with ties, -inf and NaN, and rows with fewer than 16 non-NaN tokens. */
void jfo_draft_top16(const float *row, uint32_t vocabulary, uint32_t *ids,
                     float *values) {
  for (uint32_t i = 0; i < JFO_DRAFT_CANDIDATES; ++i) {
    values[i] = -INFINITY;
    ids[i] = JFO_NO_TOKEN;
  }
  for (uint32_t t = 0; t < vocabulary; ++t) {
    const float v = row[t];
    const uint32_t last = JFO_DRAFT_CANDIDATES - 1;
    if (!draft_beats(v, t, values[last], ids[last]))
      continue;
    uint32_t slot = last;
    while (slot > 0 && draft_beats(v, t, values[slot - 1], ids[slot - 1])) {
      values[slot] = values[slot - 1];
      ids[slot] = ids[slot - 1];
      --slot;
    }
    values[slot] = v;
    ids[slot] = t;
  }
}

static float bf16f(uint16_t b) { return u2f((uint32_t)b << 16); }

/* Pinned by tests/test_oracle.py against float64 dot products (and by the
 * roles: swapping the codebooks or dropping the hidden factor fails it). */
float jfo_draft_edge(const uint16_t *pred_row, const uint16_t *hidden,
                     const uint16_t *succ_row) {
  float acc = 0.0f;
  for (uint32_t d = 0; d < JFO_DRAFT_RANK; ++d) {
    const float context = bf16f(pred_row[d]) * bf16f(hidden[d]);
    acc = acc + context * bf16f(succ_row[d]);
  }
  return acc;
}

/* draft_select_top16_sharded + draft_select_edges + draft_select_dflash for
 * one lane. The walk is pinned by tests/test_oracle.py: greedy against a
 * numpy argmax chain, sampled q against a float64 softmax. */
void jfo_draft_select_lane(const jfo_draft_lane *lane, const float *logits8,
                           uint64_t stride, const uint16_t *hidden8,
                           const uint16_t *pred_codebook,
                           const uint16_t *succ_codebook,
                           const float *uniforms40, uint32_t *candidates,
                           float *unary, uint32_t *tokens, float *q) {
  const uint32_t V = lane->vocabulary, K = JFO_DRAFT_CANDIDATES;
  for (uint32_t p = 0; p < JFO_DRAFT_POSITIONS; ++p)
    jfo_draft_top16(logits8 + (uint64_t)(p + 1) * stride, V, candidates + p * K,
                    unary + p * K);
  /* Edge tables: position p scores predecessor i (the anchor at p = 0, row
   * p - 1's candidate i after) against candidate j (sampling.metal:1233-1288;
   * ids are clamped into the codebooks as there). */
  float table[JFO_DRAFT_POSITIONS][JFO_DRAFT_CANDIDATES][JFO_DRAFT_CANDIDATES];
  for (uint32_t p = 0; p < JFO_DRAFT_POSITIONS; ++p) {
    const uint16_t *h = hidden8 + (uint64_t)(p + 1) * JFO_DRAFT_RANK;
    const uint32_t preds = p ? K : 1;
    for (uint32_t i = 0; i < preds; ++i) {
      uint32_t pred = p ? candidates[(p - 1) * K + i] : lane->anchor;
      pred = pred < V - 1 ? pred : V - 1;
      for (uint32_t j = 0; j < K; ++j) {
        uint32_t c = candidates[p * K + j];
        c = c < V - 1 ? c : V - 1;
        table[p][i][j] = jfo_draft_edge(pred_codebook + (uint64_t)pred * JFO_DRAFT_RANK, h,
                                        succ_codebook + (uint64_t)c * JFO_DRAFT_RANK);
      }
    }
  }
  /* The walk (sampling.metal:1316-1359). */
  uint32_t pred_index = 0;
  for (uint32_t p = 0; p < JFO_DRAFT_POSITIONS; ++p) {
    float scores[JFO_DRAFT_CANDIDATES];
    for (uint32_t i = 0; i < K; ++i)
      scores[i] = unary[p * K + i] + table[p][pred_index][i];
    uint32_t selected = 0;
    if (lane->sampled) {
      float maximum = scores[0];
      for (uint32_t i = 1; i < K; ++i)
        maximum = fmaxf(maximum, scores[i]);
      float prob[JFO_DRAFT_CANDIDATES], sum = 0.0f;
      for (uint32_t i = 0; i < K; ++i) {
        prob[i] = jfo_expf((scores[i] - maximum) / lane->temperature);
        sum = sum + prob[i];
      }
      float cumulative = 0.0f;
      selected = K - 1;
      for (uint32_t i = 0; i < K; ++i) {
        const float pi = prob[i] / sum;
        q[p * K + i] = pi;
        cumulative = cumulative + pi;
        if (selected == K - 1 && cumulative > uniforms40[1 + p])
          selected = i;
      }
    } else {
      for (uint32_t i = 1; i < K; ++i)
        if (scores[i] > scores[selected])
          selected = i;
    }
    pred_index = selected;
    tokens[p] = candidates[p * K + selected];
  }
}

/* ---- tree gather --------------------------------------------------------- */

/* verify_tree_gather (tree.metal:86-107), one column at a time. Pinned by
 * tests/test_oracle.py against the closed form row i := original row
 * path[i] (i < retained), other rows unchanged. */
void jfo_tree_gather(uint16_t *data, const uint32_t *path_rows,
                     const uint32_t *retained, const jfo_gather_params *p) {
  for (uint32_t b = 0; b < p->lanes; ++b) {
    uint32_t rows = retained[b] < JFO_TREE_MAX_DEPTH ? retained[b] : JFO_TREE_MAX_DEPTH;
    for (uint32_t y = 0; y < p->layers; ++y)
      for (uint32_t c = 0; c < p->columns; ++c) {
        const uint64_t base = (uint64_t)y * p->layer_stride + (uint64_t)b * p->lane_stride +
                              (uint64_t)(c / p->inner) * p->outer_stride +
                              (uint64_t)(c % p->inner) * p->inner_stride;
        for (uint32_t i = 0; i < rows; ++i) {
          const uint32_t src = path_rows[b * JFO_TREE_MAX_DEPTH + i];
          if (src != i && src < p->rows)
            data[base + (uint64_t)i * p->row_stride] = data[base + (uint64_t)src * p->row_stride];
        }
      }
  }
}
