// justfit::hip::Sampling — the reference's target token policy operator
// (source/runtime/ops/Sampling.hpp:13-199) over HIP device buffers, built on
// the C ABI of include/jf_sampler.h. Same policy types, method names,
// argument meaning and exceptions; a CommandGraph is replaced by the HIP
// stream the work is enqueued on, a MetalBuffer by a device pointer and its
// size.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <optional>
#include <span>
#include <vector>

#include "jf_sampler.h"

namespace justfit::hip {

// Sampling.hpp:19-27
struct SamplingPenalties final {
  float repetition = 1.0F;
  float presence = 0.0F;
  float frequency = 0.0F;
  [[nodiscard]] bool active() const noexcept {
    return repetition != 1.0F || presence != 0.0F || frequency != 0.0F;
  }
};

// Sampling.hpp:31-50
struct SamplingPolicy final {
  uint32_t topK = 0;
  float temperature = 0.0F;
  float topP = 1.0F;
  bool constrained = false;
  bool excludesStopTokens = false;
  SamplingPenalties penalties{};
  float minP = 0.0F;
  [[nodiscard]] bool samples() const noexcept { return temperature > 0.0F; }
};

// A device allocation (the MetalBuffer role).
struct DeviceBuffer final {
  void *data = nullptr;
  uint64_t sizeBytes = 0;
};

// Sampling.hpp:55-58: the penalty words of every state lane and the row
// each lane of a dispatch reads.
struct PenaltyTable final {
  jf_penalty_table *words = nullptr;
  std::span<const uint32_t> rows;
};

// Sampling.hpp:69-97, the buffers a selection touches. Scratch the reference
// passes in (partial masses, argmax partials, ranges, arrivals) is owned by
// the operator. draftProbabilities is one float per selected row (the
// draft_probability field of the reference's TargetVocabularyRow).
struct SamplingBuffers final {
  DeviceBuffer logits;            // fp32 [lanes * verifyRows][vocabulary]
  DeviceBuffer uniforms;          // fp32 [lanes][40]
  DeviceBuffer constraintMasks;   // u32 [lanes * (verifyRows + 1)][words]
  DeviceBuffer outputTokens;      // u32 [lanes * rows]
  DeviceBuffer inputTokens;       // u32 [lanes * verifyRows]
  DeviceBuffer draftCandidates;   // u32 [lanes * (verifyRows - 1)][16]
  DeviceBuffer draftProbabilities;// f32 [lanes * (verifyRows - 1)][16]
  DeviceBuffer targetProbabilities; // f32 [lanes * verifyRows]
};

// Sampling.hpp:99-108
struct AcceptanceBuffers final {
  DeviceBuffer proposedTokens;
  DeviceBuffer candidates;
  DeviceBuffer proposalProbabilities;
  DeviceBuffer targetProbabilities;
  DeviceBuffer uniforms;
  DeviceBuffer outputTokens;
  DeviceBuffer retainedCounts;
  DeviceBuffer acceptedCounts;
};

// ops/VerifyShape.hpp:6-18: verify rows per lane, 8 or 16, per thread.
uint32_t activeVerifyRows() noexcept;
class VerifyShapeScope {
 public:
  explicit VerifyShapeScope(uint32_t rows);
  ~VerifyShapeScope();
  VerifyShapeScope(const VerifyShapeScope &) = delete;
  VerifyShapeScope &operator=(const VerifyShapeScope &) = delete;

 private:
  uint32_t prior_;
};

class Sampling final {
 public:
  // Sampling.cpp:82-86; the operator also owns the device scratch of up to
  // maximumLanes * 16 selected rows.
  explicit Sampling(uint32_t vocabulary, uint32_t maximumLanes = 4);
  ~Sampling();
  Sampling(const Sampling &) = delete;
  Sampling &operator=(const Sampling &) = delete;

  static void rebuildPenaltyWords(std::span<uint32_t> words,
                                  std::span<const uint32_t> history,
                                  uint64_t generatedTokens,
                                  std::optional<uint32_t> pendingToken,
                                  bool markPrompt);
  static void countPenaltyTokens(std::span<uint32_t> words,
                                 std::span<const uint32_t> selected);

  void addInitial(hipStream_t stream, std::span<const SamplingPolicy> policies,
                  const SamplingBuffers &buffers, uint32_t rowOffset,
                  uint32_t stopToken0, uint32_t stopToken1,
                  const PenaltyTable &penalties) const;
  void addVerify(hipStream_t stream, std::span<const SamplingPolicy> policies,
                 const SamplingBuffers &buffers, uint32_t stopToken0,
                 uint32_t stopToken1, const PenaltyTable &penalties,
                 bool tree = false) const;
  void addAcceptance(hipStream_t stream, const AcceptanceBuffers &buffers,
                     std::span<const uint32_t> maximumRetained,
                     std::span<const SamplingPolicy> policies,
                     uint32_t stopToken0, uint32_t stopToken1) const;

  [[nodiscard]] uint32_t vocabulary() const noexcept { return vocabulary_; }

 private:
  uint32_t vocabulary_ = 0;
  uint32_t maskWords_ = 0;
  uint32_t maximumLanes_ = 0;
  jf_sampler *sampler_ = nullptr;
  // Each verify row's uniform slot (device): four tables of maximumLanes * 16
  // entries, by (tree draws or the correction slot) x (8 or 16 rows).
  uint32_t *uniformIndex_ = nullptr;
};

}  // namespace justfit::hip
