// Host-only parts of the library: the error text behind jf_last_error, and
// the host copy of the penalty table from which device updates are derived.
// Nothing here includes the HIP runtime, so these sources also build with a
// plain host compiler (and its sanitizers).
#pragma once

#include <cstdint>
#include <string>
#include <vector>

namespace jf {

// Sets jf_last_error's text for this thread; returns `code`.
int set_error(int code, const char *message);
int set_error(int code, const std::string &message);

// The fast kernel's fixed slot of one penalized token: its offset in the
// 8192-token chunk, the prompt bit and the generated count.
constexpr uint32_t kPenaltyChunk = 8192;
constexpr uint32_t kPenaltyBucket = 2048;
constexpr uint32_t kSlotCountMask = 0x3ffffu;
constexpr uint32_t kSlotPromptBit = 0x40000u;
constexpr int kSlotOffsetShift = 19;
constexpr uint32_t kNoSlot = 0xffffffffu;

// One device entry: a token and its penalty word (count | prompt bit),
// laid out as the device's {token, word} pairs.
struct PenaltyEntry {
  uint32_t token;
  uint32_t word;
};

// One counted token as the device applies it to a row, in call order:
// the entry at `index` gets `word`; with `insert` set, entries [index,
// entries) first move up one place and bucket offsets past the token's
// bucket grow by one. The slot half does the same inside the token's chunk
// (slot == kNoSlot: the row's slots are not kept, the row no longer fits).
struct PenaltyOp {
  uint32_t row;
  uint32_t token;
  uint32_t index;
  uint32_t insert;
  uint32_t word;
  uint32_t entries;     // the row's entry count before the op
  uint32_t slot;        // slot index inside the chunk
  uint32_t slot_value;  // offset << kSlotOffsetShift | prompt bit | count
  uint32_t slot_used;   // the chunk's used slots before the op
};

// Host copy of every table row: entries sorted by token, kept per 2048-token
// bucket with the buckets' running offsets (so a count costs the bucket's
// entries and one pass over the offsets, not a move of the row), and
// whether the row's chunks fit their fixed slots.
class PenaltyRows {
 public:
  void init(uint32_t vocabulary, uint32_t rows, uint32_t max_entries,
            uint32_t slot_count);
  uint32_t vocabulary() const { return vocabulary_; }
  uint32_t rows() const { return rows_; }
  uint32_t buckets() const { return buckets_; }
  uint32_t chunks() const { return chunks_; }
  uint32_t slot_count() const { return slot_count_; }
  uint32_t max_entries() const { return max_entries_; }

  // rebuildPenaltyWords' result (dense words) as row `row`. Fails, leaving
  // the row unchanged, when it holds more than max_entries tokens.
  int rebuild(uint32_t row, const uint32_t *words);
  // countPenaltyTokens of `token` on row `row`: updates the copy and
  // describes the device update. Fails, leaving the row unchanged, when a
  // new token would exceed max_entries.
  int count(uint32_t row, uint32_t token, PenaltyOp *op);

  uint32_t size(uint32_t row) const { return offsets_[row][buckets_]; }
  bool holds(uint32_t row, uint32_t token) const;
  // Starts the loads a count of `token` on row `row` will make (its bucket's
  // entries and the row's offsets), so that a batch of counts over many
  // rows overlaps their cache misses.
  void prefetch(uint32_t row, uint32_t token) const;
  bool fits(uint32_t row) const { return fits_[row] != 0; }
  // Whether the row would fit chunks of n slots.
  bool fits_at(uint32_t row, uint32_t n) const;
  // Lays the slots out n to a chunk from now on and decides again which
  // rows fit.
  void set_slot_count(uint32_t n);
  // The row as the device holds it: its entries in token order, its bucket
  // offsets (buckets + 1 values: the index of each bucket's first entry),
  // and its fixed slots (chunks x slot_count values, empty slots 0).
  void entries(uint32_t row, PenaltyEntry *out) const;
  void offsets(uint32_t row, uint32_t *out) const;
  void slots(uint32_t row, uint32_t *out) const;

 private:
  static uint32_t slot_value(const PenaltyEntry &e);
  void refit(uint32_t row);

  uint32_t vocabulary_ = 0, rows_ = 0, max_entries_ = 0;
  uint32_t buckets_ = 0, chunks_ = 0, slot_count_ = 0;
  std::vector<std::vector<std::vector<PenaltyEntry>>> bucket_;  // [row][bucket]
  std::vector<std::vector<uint32_t>> offsets_;                  // [row][buckets + 1]
  std::vector<uint8_t> fits_;
};

}  // namespace jf
