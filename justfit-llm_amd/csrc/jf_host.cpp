// Host-only entry points of the C ABI (include/jf_sampler.h) and the host
// copy of the penalty table: error text, policy validation, the dense
// penalty-word helpers, SplitMix64 uniforms, and the per-row sorted entries
// and fixed slots from which device updates are derived.
#include "jf_host.h"

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <utility>

#include "jf_sampler.h"

namespace {
thread_local std::string g_error;
}  // namespace

namespace jf {

int set_error(int code, const char *message) {
  g_error = message;
  return code;
}

int set_error(int code, const std::string &message) {
  g_error = message;
  return code;
}

static_assert(kPenaltyChunk % kPenaltyBucket == 0, "a chunk is whole buckets");
constexpr uint32_t kBucketsPerChunk = kPenaltyChunk / kPenaltyBucket;

void PenaltyRows::init(uint32_t vocabulary, uint32_t rows, uint32_t max_entries,
                       uint32_t slot_count) {
  vocabulary_ = vocabulary;
  rows_ = rows;
  max_entries_ = max_entries;
  buckets_ = (vocabulary + kPenaltyBucket - 1) / kPenaltyBucket;
  chunks_ = (vocabulary + kPenaltyChunk - 1) / kPenaltyChunk;
  slot_count_ = slot_count;
  bucket_.assign(rows, std::vector<std::vector<PenaltyEntry>>(buckets_));
  offsets_.assign(rows, std::vector<uint32_t>(buckets_ + 1, 0u));
  fits_.assign(rows, 1);
}

uint32_t PenaltyRows::slot_value(const PenaltyEntry &e) {
  return ((e.token % kPenaltyChunk) << kSlotOffsetShift) |
         ((e.word & JF_PENALTY_PROMPT_BIT) ? kSlotPromptBit : 0u) |
         (e.word & JF_PENALTY_COUNT_MASK);
}

// Whether every chunk fits n slots with every count inside the slot's
// count field.
bool PenaltyRows::fits_at(uint32_t row, uint32_t n) const {
  const std::vector<uint32_t> &off = offsets_[row];
  for (uint32_t c = 0; c < chunks_; ++c) {
    const uint32_t b0 = c * kBucketsPerChunk;
    const uint32_t b1 = std::min(b0 + kBucketsPerChunk, buckets_);
    if (off[b1] - off[b0] > n) return false;
  }
  for (uint32_t b = 0; b < buckets_; ++b)
    for (const PenaltyEntry &e : bucket_[row][b])
      if ((e.word & JF_PENALTY_COUNT_MASK) > kSlotCountMask) return false;
  return true;
}

void PenaltyRows::refit(uint32_t row) { fits_[row] = fits_at(row, slot_count_) ? 1 : 0; }

void PenaltyRows::set_slot_count(uint32_t n) {
  slot_count_ = n;
  for (uint32_t r = 0; r < rows_; ++r) refit(r);
}

int PenaltyRows::rebuild(uint32_t row, const uint32_t *words) {
  uint64_t n = 0;
  for (uint32_t v = 0; v < vocabulary_; ++v) n += words[v] != 0;
  if (n > max_entries_)
    return set_error(JF_ERR_INVALID_ARGUMENT, "penalty history exceeds the table row");
  std::vector<std::vector<PenaltyEntry>> &bk = bucket_[row];
  std::vector<uint32_t> &off = offsets_[row];
  uint32_t total = 0;
  for (uint32_t b = 0; b < buckets_; ++b) {
    bk[b].clear();
    off[b] = total;
    const uint32_t end = std::min((b + 1) * kPenaltyBucket, vocabulary_);
    for (uint32_t v = b * kPenaltyBucket; v < end; ++v)
      if (words[v]) bk[b].push_back({v, words[v]});
    total += (uint32_t)bk[b].size();
  }
  off[buckets_] = total;
  refit(row);
  return JF_OK;
}

bool PenaltyRows::holds(uint32_t row, uint32_t token) const {
  const std::vector<PenaltyEntry> &v = bucket_[row][token / kPenaltyBucket];
  const auto it = std::lower_bound(
      v.begin(), v.end(), token,
      [](const PenaltyEntry &e, uint32_t t) { return e.token < t; });
  return it != v.end() && it->token == token;
}

void PenaltyRows::prefetch(uint32_t row, uint32_t token) const {
  const uint32_t b = token / kPenaltyBucket;
  const std::vector<PenaltyEntry> &v = bucket_[row][b];
  const PenaltyEntry *d = v.data();
  for (size_t k = 0; k < v.size(); k += 8) __builtin_prefetch(d + k);
  const uint32_t *off = offsets_[row].data();
  for (uint32_t k = b; k <= buckets_; k += 16) __builtin_prefetch(off + k);
  __builtin_prefetch(off + (token / kPenaltyChunk) * kBucketsPerChunk);
}

int PenaltyRows::count(uint32_t row, uint32_t token, PenaltyOp *op) {
  const uint32_t b = token / kPenaltyBucket;
  std::vector<PenaltyEntry> &v = bucket_[row][b];
  std::vector<uint32_t> &off = offsets_[row];
  const auto it = std::lower_bound(
      v.begin(), v.end(), token,
      [](const PenaltyEntry &e, uint32_t t) { return e.token < t; });
  const bool found = it != v.end() && it->token == token;
  if (!found && off[buckets_] >= max_entries_)
    return set_error(JF_ERR_INVALID_ARGUMENT, "penalty history exceeds the table row");
  const uint32_t index = off[b] + (uint32_t)(it - v.begin());
  op->row = row;
  op->token = token;
  op->index = index;
  op->insert = found ? 0u : 1u;
  op->entries = off[buckets_];
  // Sampling.cpp:75-80: the word's count grows by one (the prompt bit stays).
  const uint32_t word = found ? it->word + 1u : 1u;
  op->word = word;
  // The token's chunk before the op: its first entry and its used slots.
  const uint32_t c = token / kPenaltyChunk;
  const uint32_t b0 = c * kBucketsPerChunk, b1 = std::min(b0 + kBucketsPerChunk, buckets_);
  const uint32_t first = off[b0], used = off[b1] - off[b0];
  if (found) {
    it->word = word;
  } else {
    v.insert(it, PenaltyEntry{token, word});
    for (uint32_t k = b + 1; k <= buckets_; ++k) ++off[k];
  }
  op->slot = kNoSlot;
  op->slot_value = 0;
  op->slot_used = 0;
  if (fits_[row]) {
    if ((!found && used >= slot_count_) || (word & JF_PENALTY_COUNT_MASK) > kSlotCountMask) {
      // The row stops fitting: the fast kernel no longer takes it, and its
      // slots are rebuilt only by a rebuild that fits again.
      fits_[row] = 0;
    } else {
      op->slot = index - first;
      op->slot_value = slot_value(PenaltyEntry{token, word});
      op->slot_used = used;
    }
  }
  return JF_OK;
}

void PenaltyRows::entries(uint32_t row, PenaltyEntry *out) const {
  for (uint32_t b = 0; b < buckets_; ++b)
    for (const PenaltyEntry &e : bucket_[row][b]) *out++ = e;
}

void PenaltyRows::offsets(uint32_t row, uint32_t *out) const {
  std::copy(offsets_[row].begin(), offsets_[row].end(), out);
}

void PenaltyRows::slots(uint32_t row, uint32_t *out) const {
  std::fill(out, out + (size_t)chunks_ * slot_count_, 0u);
  for (uint32_t c = 0; c < chunks_; ++c) {
    uint32_t used = 0;
    const uint32_t b1 = std::min((c + 1) * kBucketsPerChunk, buckets_);
    for (uint32_t b = c * kBucketsPerChunk; b < b1; ++b)
      for (const PenaltyEntry &e : bucket_[row][b])
        if (used < slot_count_) out[(size_t)c * slot_count_ + used++] = slot_value(e);
  }
}

}  // namespace jf

extern "C" {

const char *jf_last_error(void) { return g_error.c_str(); }

int jf_policy_validate(const jf_policy *p) {
  if (!p) return jf::set_error(JF_ERR_INVALID_ARGUMENT, "policy is null");
  const bool temperature_valid =
      p->temperature == 0.0f ||
      (std::isfinite(p->temperature) && p->temperature >= FLT_MIN);
  if (!temperature_valid || !(p->top_p > 0.0f && p->top_p <= 1.0f) ||
      !(p->min_p >= 0.0f) || p->min_p > 1.0f)
    return jf::set_error(JF_ERR_INVALID_ARGUMENT,
                         "sampling requires temperature 0 or at least FLT_MIN, top_p "
                         "in (0,1] and min_p in [0,1]");
  if (!(std::fabs(p->presence) <= 2.0f) || !(std::fabs(p->frequency) <= 2.0f) ||
      !std::isfinite(p->repetition) || p->repetition <= 0.0f)
    return jf::set_error(JF_ERR_INVALID_ARGUMENT,
                         "sampling requires presence and frequency penalties in [-2,2] "
                         "and a positive repetition penalty");
  return JF_OK;
}

int jf_penalty_words_rebuild(uint32_t *words, uint32_t vocabulary,
                             const uint32_t *history, uint64_t history_len,
                             uint64_t generated, int has_pending,
                             uint32_t pending, int mark_prompt) {
  if (history_len <= generated)
    return jf::set_error(JF_ERR_LOGIC, "request history holds no prompt");
  if ((!words && vocabulary) || (!history && history_len))
    return jf::set_error(JF_ERR_INVALID_ARGUMENT, "null buffer");
  for (uint64_t i = 0; i < history_len; ++i)
    if (history[i] >= vocabulary)
      return jf::set_error(JF_ERR_INVALID_ARGUMENT, "penalty token is outside the vocabulary");
  if (has_pending && pending >= vocabulary)
    return jf::set_error(JF_ERR_INVALID_ARGUMENT, "penalty token is outside the vocabulary");
  const uint64_t prompt = history_len - generated;
  std::fill(words, words + vocabulary, 0u);
  if (mark_prompt)
    for (uint64_t i = 0; i < prompt; ++i) words[history[i]] |= JF_PENALTY_PROMPT_BIT;
  for (uint64_t i = prompt; i < history_len; ++i) ++words[history[i]];
  if (has_pending) ++words[pending];
  return JF_OK;
}

int jf_penalty_words_count(uint32_t *words, uint32_t vocabulary,
                           const uint32_t *selected, uint64_t count) {
  if ((!selected && count) || (!words && vocabulary))
    return jf::set_error(JF_ERR_INVALID_ARGUMENT, "null buffer");
  for (uint64_t i = 0; i < count; ++i)
    if (selected[i] >= vocabulary)
      return jf::set_error(JF_ERR_INVALID_ARGUMENT, "penalty token is outside the vocabulary");
  for (uint64_t i = 0; i < count; ++i) ++words[selected[i]];
  return JF_OK;
}

float jf_next_uniform(uint64_t seed, uint64_t *counter) {
  uint64_t v = seed + (++*counter) * 0x9e3779b97f4a7c15ULL;
  v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ULL;
  v = (v ^ (v >> 27)) * 0x94d049bb133111ebULL;
  v ^= v >> 31;
  return float(v >> 40) * 0x1p-24F;
}

void jf_stage_sampling_cycle(uint64_t seed, uint64_t *counter,
                             uint32_t verify_rows, int tree_cycle,
                             float *u) {
  std::fill(u, u + JF_SAMPLING_UNIFORMS, 0.0f);
  const uint32_t end = (tree_cycle && verify_rows == 16) ? JF_SAMPLING_UNIFORMS
                       : verify_rows == 16                ? 24u
                                                          : 16u;
  for (uint32_t i = JF_UNIFORM_PROPOSALS; i < end; ++i)
    u[i] = jf_next_uniform(seed, counter);
}

}  // extern "C"
